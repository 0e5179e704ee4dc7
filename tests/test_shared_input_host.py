"""Host-side checks of the shared-input groups (drinkme_amd/swap.py:
SharedInputGroup, install_groups) that need no GPU: which sibling modules
install_groups joins, and when a member's call reuses the grouped launch of
an earlier member's call and when it launches again. The launch itself is
replaced by a counter that returns a fresh tensor per member; its GPU parity
is in tests/test_gpu_group.py."""

import pytest
import torch

from drinkme_amd import radix_ops, swap


def _fake_runtime(R, C, device="cpu"):
    """The fields a module and a group read before any launch."""
    return {"codec": "radix", "R": R, "C": C, "rx_data": torch.zeros(4, dtype=torch.int32, device=device)}


def _module(R, C, bias=None):
    return swap.RadixCompressedLinear(_fake_runtime(R, C), bias)


class _Attn(torch.nn.Module):
    def __init__(self, C=64, kv=16, bias=None):
        super().__init__()
        self.q_proj, self.k_proj, self.v_proj = _module(C, C, bias), _module(kv, C), _module(kv, C)
        self.o_proj = _module(C, C)


class _Mlp(torch.nn.Module):
    def __init__(self, C=64, F=128):
        super().__init__()
        self.gate_proj, self.up_proj, self.down_proj = _module(F, C), _module(F, C), _module(C, F)


class _Layer(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.self_attn, self.mlp = _Attn(), _Mlp()


def test_install_groups_joins_qkv_and_gate_up_per_layer():
    model = torch.nn.ModuleDict({"layers": torch.nn.ModuleList([_Layer(), _Layer()])})
    made = swap.install_groups(model)
    assert made == [("layers.0.self_attn.q_proj", "layers.0.self_attn.k_proj", "layers.0.self_attn.v_proj"),
                    ("layers.0.mlp.gate_proj", "layers.0.mlp.up_proj"),
                    ("layers.1.self_attn.q_proj", "layers.1.self_attn.k_proj", "layers.1.self_attn.v_proj"),
                    ("layers.1.mlp.gate_proj", "layers.1.mlp.up_proj")]
    a = model["layers"][0].self_attn
    assert a.q_proj._group is a.k_proj._group is a.v_proj._group is not None
    assert [a.q_proj._slot, a.k_proj._slot, a.v_proj._slot] == [0, 1, 2]
    assert a.o_proj._group is None and model["layers"][0].mlp.down_proj._group is None
    assert a.q_proj._group is not model["layers"][1].self_attn.q_proj._group
    assert swap.install_groups(model) == []  # grouped modules are not grouped again


def test_install_groups_skips_what_one_launch_cannot_serve():
    attn = _Attn()
    attn.v_proj = torch.nn.Linear(64, 16)  # not a radix module: q and k still group
    assert swap.install_groups(attn) == [("q_proj", "k_proj")]
    odd = _Attn()
    odd.k_proj = _module(16, 128)  # another column count: not one activation, nothing grouped
    assert swap.install_groups(odd) == []
    mixed = _Attn(bias=torch.zeros(64, dtype=torch.bfloat16))
    mixed.k_proj.bias = torch.zeros(16, dtype=torch.float32)  # biases the kernel cannot take in one launch
    assert swap.install_groups(mixed) == []
    lone = torch.nn.Module()
    lone.q_proj = _module(64, 64)
    assert swap.install_groups(lone) == []


def test_group_refusals():
    a, b = _module(8, 64), _module(8, 64)
    with pytest.raises(ValueError, match="at least two"):
        swap.SharedInputGroup([a])
    with pytest.raises(ValueError, match="twice"):
        swap.SharedInputGroup([a, a])
    with pytest.raises(TypeError, match="not a RadixCompressedLinear"):
        swap.SharedInputGroup([a, torch.nn.Linear(64, 8)])
    with pytest.raises(ValueError, match="C = 64"):
        swap.SharedInputGroup([a, _module(8, 32)])
    g = swap.SharedInputGroup([a, b])
    with pytest.raises(ValueError, match="already in a group"):
        swap.SharedInputGroup([b, _module(8, 64)])
    g.dissolve()
    assert a._group is None and b._group is None
    swap.SharedInputGroup([b, _module(8, 64)])


@pytest.fixture
def counted(monkeypatch):
    """A three-member group whose launch counts its calls and returns one
    fresh tensor per member, tagged with the launch's number."""
    monkeypatch.setattr(radix_ops, "_stream", lambda device=None: 7)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    mods = [_module(R, 64) for R in (64, 16, 16)]
    g = swap.SharedInputGroup(mods)
    calls = []

    def launch(rows, biases, dtype):
        calls.append((rows.numel() // 64, dtype))
        n = len(calls)
        return [torch.full((*rows.shape[:-1], R), float(n), dtype=dtype) for R in (64, 16, 16)]

    g.launch = launch
    return g, calls


def _x(m=1, dtype=torch.bfloat16):
    return torch.randn(m, 64).to(dtype)


def test_one_launch_serves_every_member_once(counted):
    g, calls = counted
    x = _x()
    ys = [g.rows(slot, x) for slot in (0, 1, 2)]
    assert len(calls) == 1 and [tuple(y.shape) for y in ys] == [(1, 64), (1, 16), (1, 16)]
    assert g._x is None, "the activation is released once every member has its rows"
    # the same members again on the same activation: a new step, a new launch
    ys = [g.rows(slot, x) for slot in (2, 0, 1)]
    assert len(calls) == 2 and all(float(y[0, 0]) == 2.0 for y in ys)


def test_a_member_called_twice_launches_again(counted):
    g, calls = counted
    x = _x()
    g.rows(0, x)
    y = g.rows(0, x)
    assert len(calls) == 2 and float(y[0, 0]) == 2.0
    assert float(g.rows(1, x)[0, 0]) == 2.0 and len(calls) == 2


def test_an_in_place_write_between_members_launches_again(counted):
    g, calls = counted
    x = _x()
    g.rows(0, x)
    x.mul_(2)  # torch bumps the version counter
    y = g.rows(1, x)
    assert len(calls) == 2 and float(y[0, 0]) == 2.0


def test_another_tensor_with_the_same_values_launches_again(counted):
    g, calls = counted
    x = _x()
    g.rows(0, x)
    twin = x.clone()
    g.rows(1, twin)
    assert len(calls) == 2
    view = x.view(1, 64)  # another object over the same memory: launches too
    g.rows(2, view)
    assert len(calls) == 3


def test_stream_and_capture_state_are_part_of_the_match(counted, monkeypatch):
    g, calls = counted
    x = _x()
    g.rows(0, x)
    monkeypatch.setattr(radix_ops, "_stream", lambda device=None: 8)
    g.rows(1, x)
    assert len(calls) == 2
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    g.rows(2, x)
    assert len(calls) == 3


def test_inference_tensors_match_by_identity(counted):
    g, calls = counted
    with torch.inference_mode():
        x = _x()
        ys = [g.rows(slot, x) for slot in (0, 1, 2)]
    assert len(calls) == 1 and len(ys) == 3


def test_reset_drops_the_held_rows(counted):
    g, calls = counted
    x = _x()
    g.rows(0, x)
    g.reset()
    g.rows(1, x)
    assert len(calls) == 2


def test_the_launch_gets_the_members_biases_and_x_dtype(monkeypatch):
    monkeypatch.setattr(radix_ops, "_stream", lambda device=None: 7)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    bq = torch.ones(64, dtype=torch.float32)
    mods = [_module(64, 64, bq), _module(16, 64)]
    g = swap.SharedInputGroup(mods)
    seen = []
    g.launch = lambda rows, biases, dtype: seen.append((biases, dtype)) or [torch.zeros(1, 64), torch.zeros(1, 16)]
    x = _x(dtype=torch.float32)
    g.rows(1, x)
    (biases, dtype), = seen
    assert biases[0] is bq and biases[1] is None and dtype == torch.float32


def test_new_storage_under_the_same_activation_launches_again(counted):
    g, calls = counted
    x = _x()
    g.rows(0, x)
    x.data = x.data.clone()  # the same object over new memory, its version untouched
    g.rows(1, x)
    assert len(calls) == 2


def test_the_bias_array_follows_the_biases_addresses():
    from drinkme_amd import radix_ops

    gl = radix_ops.GroupLauncher([_fake_runtime(8, 64), _fake_runtime(4, 64)])
    x = torch.zeros(1, 64, dtype=torch.bfloat16)
    b = torch.ones(8, dtype=torch.bfloat16)
    arr, bd, kept = gl._bias_array([b, None], x)
    assert arr[0] == b.data_ptr() and arr[1] is None
    assert gl._bias_array([b, None], x)[0] is arr, "the same biases at the same addresses: the cached array"
    b.data = torch.full((8,), 2.0, dtype=torch.bfloat16)  # new storage under the same Parameter-like tensor
    arr2 = gl._bias_array([b, None], x)[0]
    assert arr2 is not arr and arr2[0] == b.data_ptr()
    wide = torch.ones(16, dtype=torch.bfloat16)[::2]  # not contiguous: copied for the call, never cached
    arr3, _, kept3 = gl._bias_array([wide, None], x)
    assert arr3[0] == kept3[0].data_ptr() != wide.data_ptr()
    assert gl._bias_array([wide, None], x)[0] is not arr3
