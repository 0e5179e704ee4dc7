"""GPU: the raw bf16 GEMV (dmx_gemv_narrow) through the C ABI — drinkme's
_gemv_narrow (src/drinkme/codec/radix_ops.py:177-249) as swap.NarrowLinear
runs it, and the twin route of the GEMV calls (radix_ops.py:252-255).

Against the float64 oracle (within 2e-6 |x|.|W| + 1e-7), and what drinkme's
tests/test_narrow_linear.py pins on the GPU: the bias added in fp32 before
the one rounding (the 2^-9 known answer), row m of an M-row call equal to
the one-row call bit for bit on the three narrow shapes, a bf16 x giving
the bits of its fp32 widening, M > 8 being F.linear, install_narrow
adopting exactly the sub-threshold Linears. Ragged and unaligned inputs
take the element-load path, whose sums are the vector path's bit for bit.
"""

import numpy as np
import pytest

from oracle import radix_oracle as O
from tests.helpers import bf16_tensor, finite_bits

pytestmark = pytest.mark.gpu


def _check(y, xf, bits, what):
    ref, bound = O.gemv_f64(bits, xf)
    err = np.abs(np.asarray(y, np.float64).reshape(ref.shape) - ref) / bound
    assert np.all(err <= 1.0), f"{what}: err/bound {err.max():.3f}"


@pytest.mark.parametrize("R,C", [(48, 5120), (32, 4096), (256, 6656), (7, 1000), (1, 12), (300, 1032), (5, 25600)])
@pytest.mark.parametrize("M", [1, 3, 8])
def test_narrow_matches_the_oracle(cuda, R, C, M):
    import torch

    from drinkme_amd import radix_ops

    rng = np.random.default_rng(R * 1000003 + C * 31 + M)
    bits = finite_bits(rng, (R, C), spread=True)
    w = bf16_tensor(bits, cuda)
    xb = O.f32_to_bf16_bits(rng.standard_normal((M, C)).astype(np.float32))
    x = bf16_tensor(xb, cuda)
    xf = O.bf16_bits_to_f32(xb)
    print(f"case narrow R={R} C={C} M={M}", flush=True)
    y = radix_ops._raw_rows(w, x, None, torch.float32, "test")
    _check(y.cpu().numpy(), xf, bits, f"narrow {R}x{C} M={M}")
    # fp32 x: the same sums bit for bit (the widening is exact)
    y32 = radix_ops._raw_rows(w, x.float(), None, torch.float32, "test")
    assert torch.equal(y32, y)
    # the bias in fp32 before the one bf16 rounding
    bias = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal(R).astype(np.float32)), cuda)
    yb = radix_ops.gemv_narrow(w, x, bias)
    assert yb.dtype == torch.bfloat16 and yb.shape == (M, R)
    assert torch.equal(yb, (y + bias.float()).to(torch.bfloat16))


def test_unaligned_activation_takes_the_element_path_with_the_same_sums(cuda):
    import torch

    from drinkme_amd import radix_ops

    rng = np.random.default_rng(9)
    R, C = 64, 4096
    w = bf16_tensor(finite_bits(rng, (R, C)), cuda)
    big = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal(C + 1).astype(np.float32)), cuda)
    x_off = big[1:].reshape(1, C)  # 2 bytes past a 16-byte boundary
    assert x_off.data_ptr() % 16 != 0
    x_al = x_off.clone()
    assert x_al.data_ptr() % 16 == 0
    a = radix_ops._raw_rows(w, x_off, None, torch.float32, "test")
    b = radix_ops._raw_rows(w, x_al, None, torch.float32, "test")
    assert torch.equal(a, b)


def _lin(r, c, cuda, bias=False, seed=0):
    import torch

    torch.manual_seed(seed)
    lin = torch.nn.Linear(c, r, bias=bias).to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.mul_(0.05)
        if bias:
            lin.bias.mul_(0.5)
    return lin.to(cuda)


@pytest.mark.parametrize("bias", [False, True])
def test_narrow_linear_vs_flinear_and_fp64(cuda, bias):
    import torch
    import torch.nn.functional as F

    from drinkme_amd import swap

    lin = _lin(48, 5120, cuda, bias=bias)
    n = swap.NarrowLinear.adopt(lin)
    torch.manual_seed(1)
    for m in (1, 5, 8):
        x = (torch.randn(m, 5120, device=cuda) * 0.5).to(torch.bfloat16)
        y = n(x)
        ref = F.linear(x, lin.weight, lin.bias)
        ref64 = x.double() @ lin.weight.double().T + (lin.bias.double() if bias else 0)
        assert y.shape == ref.shape and y.dtype == torch.bfloat16
        assert (y.float() - ref.float()).abs().max().item() < 2e-2
        assert (y.double() - ref64).abs().max().item() <= (ref.double() - ref64).abs().max().item() * 2 + 1e-3


@pytest.mark.parametrize("shape", [(48, 5120), (32, 4096), (256, 6656)])
def test_rows_of_an_m_call_equal_the_one_row_call_bitwise(cuda, shape):
    import torch

    from drinkme_amd import swap

    r, c = shape
    n = swap.NarrowLinear.adopt(_lin(r, c, cuda, bias=True))
    torch.manual_seed(2)
    x = (torch.randn(8, c, device=cuda) * 0.5).to(torch.bfloat16)
    ones = [n(x[j:j + 1]) for j in range(8)]
    for m in range(1, 9):
        ym = n(x[:m])
        for j in range(m):
            assert torch.equal(ym[j:j + 1], ones[j]), (shape, m, j)


def test_bf16_x_equals_fp32_x_bitwise(cuda):
    import torch

    from drinkme_amd import swap

    n = swap.NarrowLinear.adopt(_lin(48, 5120, cuda))
    x = (torch.randn(3, 5120, device=cuda) * 0.5).to(torch.bfloat16)
    y16, y32 = n(x), n(x.float())
    assert y16.dtype == torch.bfloat16 and y32.dtype == torch.float32
    assert torch.equal(y16.float(), y32.to(torch.bfloat16).float())


def test_bias_is_added_in_fp32_before_the_one_rounding(cuda):
    """acc 1 + 2^-9 (not a bf16 value) + bias -1 gives 2^-9, not 0."""
    import torch

    from drinkme_amd import swap

    lin = torch.nn.Linear(1024, 2, bias=True).to(torch.bfloat16).to(cuda)
    with torch.no_grad():
        lin.weight.zero_()
        lin.weight[0, 0] = 1.0
        lin.weight[0, 1] = 1.0
        lin.bias.zero_()
        lin.bias[0] = -1.0
    n = swap.NarrowLinear.adopt(lin)
    x = torch.zeros(1, 1024, dtype=torch.bfloat16, device=cuda)
    x[0, 0] = 1.0
    x[0, 1] = 2.0 ** -9
    assert n(x)[0, 0].item() == 2.0 ** -9


def test_above_mc_max_is_flinear_bitwise(cuda):
    import torch
    import torch.nn.functional as F

    from drinkme_amd import swap

    lin = _lin(48, 5120, cuda, bias=True)
    n = swap.NarrowLinear.adopt(lin)
    x = (torch.randn(9, 5120, device=cuda) * 0.5).to(torch.bfloat16)
    assert torch.equal(n(x), F.linear(x, lin.weight, lin.bias))
    x = (torch.randn(2, 40, 5120, device=cuda) * 0.5).to(torch.bfloat16)
    assert torch.equal(n(x), F.linear(x, lin.weight, lin.bias))


def test_install_narrow_adopts_exactly_the_sub_threshold_linears(cuda):
    import torch

    from drinkme_amd import swap

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.a = _lin(48, 5120, cuda)
            self.b = _lin(48, 5120, cuda, bias=True)
            self.big = _lin(1024, 5120, cuda)  # the codec's
            self.short = _lin(48, 512, cuda)  # C < MIN_COLS
            self.f32 = _lin(48, 5120, cuda).float()

    m = torch.nn.Sequential(Block(), Block())
    w_a = m[0].a.weight
    done = swap.install_narrow(m, "cuda")
    assert sorted(n for n, _ in done) == ["0.a", "0.b", "1.a", "1.b"]
    assert all(shape == (48, 5120) for _, shape in done)
    assert isinstance(m[0].a, swap.NarrowLinear) and m[0].a.weight is w_a
    assert isinstance(m[1].b, swap.NarrowLinear) and m[1].b.bias is not None
    assert type(m[0].big) is torch.nn.Linear and type(m[0].short) is torch.nn.Linear
    assert type(m[0].f32) is torch.nn.Linear
    assert swap.install_narrow(m, "cuda") == []


def test_twin_dict_runs_its_compressed_kernel_over_the_raw_weight(cuda):
    """A twin dict through the GEMV calls: within the float64 bound, the
    bias epilogue exact; its order is the compressed kernel's (pinned bit
    for bit in tests/test_gpu_twin.py)."""
    import torch

    from drinkme_amd import radix_ops, swap

    rng = np.random.default_rng(4)
    R, C = 512, 4096
    bits = finite_bits(rng, (R, C))
    twin = swap.to_device_twin(bf16_tensor(bits, cuda), device=cuda)
    xb = O.f32_to_bf16_bits(rng.standard_normal((4, C)).astype(np.float32))
    x = bf16_tensor(xb, cuda)
    y = radix_ops.gemv(twin, x[0])
    _check(y.cpu().numpy(), O.bf16_bits_to_f32(xb[:1]), bits, "twin gemv")
    mc = radix_ops.gemv_mc(twin, x)
    _check(mc.cpu().numpy(), O.bf16_bits_to_f32(xb), bits, "twin mc")
    bias = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal(R).astype(np.float32)), cuda)
    fused = radix_ops.gemv_fused(twin, x[0], bias)
    assert fused.shape == (1, R) and torch.equal(fused[0], (y + bias.float()).to(torch.bfloat16))
    grp = radix_ops.gemv_group([twin, twin], x[:2], None, torch.float32)
    two = radix_ops.gemv_mc(twin, x[:2])
    assert all(torch.equal(g, two) for g in grp)
