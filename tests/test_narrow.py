"""CPU: the raw bf16 surface of swap (NarrowLinear, install_narrow,
to_device_twin; src/drinkme/codec/swap.py:168-196, :530-627) and
gemv_narrow's argument checks, as drinkme's tests/test_narrow_linear.py
has them: what `wants` admits, `adopt` sharing the parameters, the CPU and
M > 8 fall-through being F.linear bit for bit, install_narrow a no-op off
the GPU, M outside 1..8 refused before any launch."""

import pytest
import torch
import torch.nn.functional as F

from drinkme_amd import radix_ops, swap


def _lin(r, c, bias=False, dtype=torch.bfloat16, seed=0):
    torch.manual_seed(seed)
    lin = torch.nn.Linear(c, r, bias=bias).to(dtype)
    with torch.no_grad():
        lin.weight.mul_(0.05)
        if bias:
            lin.bias.mul_(0.5)
    return lin


def test_wants_on_cpu_is_false_and_adopt_shares_parameters():
    lin = _lin(48, 5120, bias=True)
    assert not swap.NarrowLinear.wants(lin)  # a CPU weight: the kernel runs on the GPU
    n = swap.NarrowLinear.adopt(lin)
    assert isinstance(n, swap.NarrowLinear) and isinstance(n, torch.nn.Linear)
    assert n.weight is lin.weight and n.bias is lin.bias
    assert n.in_features == 5120 and n.out_features == 48
    x = torch.randn(3, 5120).to(torch.bfloat16)
    assert torch.equal(n(x), lin(x))  # the CPU fall-through is F.linear
    x = torch.randn(2, 4, 5120).to(torch.bfloat16)
    assert torch.equal(n(x), lin(x)) and n(x).shape == (2, 4, 48)


def test_install_narrow_is_a_no_op_off_the_gpu():
    m = torch.nn.Sequential(_lin(48, 5120))
    assert swap.install_narrow(m, "cpu") == []
    assert type(m[0]) is torch.nn.Linear


def test_eligible_is_the_codec_threshold():
    assert swap.eligible(_lin(1024, 1024))
    assert not swap.eligible(_lin(1023, 4096))
    assert not swap.eligible(_lin(1024, 1026))
    assert not swap.eligible(_lin(1024, 1024, dtype=torch.float32))
    assert not swap.eligible(torch.nn.Conv1d(4, 4, 1))


@pytest.mark.parametrize("m", [0, radix_ops.MC_MAX + 1])
def test_gemv_narrow_refuses_m_outside_one_to_mc_max(m):
    w = torch.zeros(48, 1024, dtype=torch.bfloat16)
    x = torch.zeros(m, 1024, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="outside 1..8"):
        radix_ops.gemv_narrow(w, x, None, 512, 4)


def test_gemv_narrow_refuses_a_non_bf16_weight():
    with pytest.raises(TypeError, match="bf16"):
        radix_ops.gemv_narrow(torch.zeros(4, 1024), torch.zeros(1, 1024), None)


def test_twin_dict_holds_the_weight_and_reads_its_bytes():
    w = _lin(64, 2048).weight.data
    with pytest.raises(TypeError, match="bf16"):
        swap.to_device_twin(w.float(), device="cpu")
    t = swap.to_device_twin(w, device="cpu")
    assert t["codec"] == "twin" and t["R"] == 64 and t["C"] == 2048 and t["NBK"] == 128
    assert torch.equal(t["weight"], w)
    assert radix_ops.read_bytes(t) == 64 * 2048 * 2


def test_fall_through_above_mc_max_is_flinear_on_cpu():
    lin = _lin(48, 5120, bias=True)
    n = swap.NarrowLinear.adopt(lin)
    x = torch.randn(radix_ops.MC_MAX + 1, 5120).to(torch.bfloat16)
    assert torch.equal(n(x), F.linear(x, lin.weight, lin.bias))
