"""GPU parity: modules joined by install_groups (drinkme_amd/swap.py), called
one by one as a decoder layer calls its q/k/v and gate/up projections.

Each module's output must be the grouped launch's (dmx_radix_gemv_group on
the same activation) bit for bit, and so within the float64 bound of the
oracle's dot over the source bits; one launch serves every member; an
in-place write between members' calls launches again; a HIP graph captured
over the members' calls replays what eager grouped launches give."""

import zlib

import numpy as np
import pytest

from oracle import radix_oracle as O
from tests.helpers import bf16_tensor, finite_bits, oracle_dict

pytestmark = pytest.mark.gpu

C, Q, KV, F = 1024, 512, 128, 1536


def _layer(cuda, profile, seed):
    """A toy decoder layer whose projections are RadixCompressedLinear over
    the oracle's packs, with a bf16 bias on q; returns it with the source
    bits of each grouped module."""
    import torch

    from drinkme_amd import swap

    rng = np.random.default_rng(seed)
    shapes = {"q_proj": (Q, C), "k_proj": (KV, C), "v_proj": (KV, C), "gate_proj": (F, C), "up_proj": (F, C)}
    bits = {n: finite_bits(rng, s, spread=(i % 2 == 1)) for i, (n, s) in enumerate(shapes.items())}
    qb = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal(Q).astype(np.float32)), cuda)
    attn, mlp = torch.nn.Module(), torch.nn.Module()
    for n in ("q_proj", "k_proj", "v_proj"):
        setattr(attn, n, swap.make_module(oracle_dict(bits[n], profile), qb if n == "q_proj" else None, cuda))
    for n in ("gate_proj", "up_proj"):
        setattr(mlp, n, swap.make_module(oracle_dict(bits[n], profile), None, cuda))
    layer = torch.nn.Module()
    layer.self_attn, layer.mlp = attn, mlp
    return layer, bits, qb


def _counting(group):
    calls = []
    inner = group.launch

    def launch(x, biases, dtype):
        calls.append(x.numel() // C)  # the activation rows of the launch
        return inner(x, biases, dtype)

    group.launch = launch
    return calls


@pytest.mark.parametrize("profile", ["sip", "gulp"])
@pytest.mark.parametrize("lead,xdt", [((1,), "bf16"), ((1, 1), "bf16"), ((4,), "bf16"), ((1, 3), "f32"),
                                      ((8,), "bf16")])
def test_members_take_one_grouped_launch(cuda, profile, lead, xdt):
    import torch

    from drinkme_amd import radix_ops, swap

    seed = zlib.crc32(repr((profile, lead, xdt)).encode())
    layer, bits, qb = _layer(cuda, profile, seed)
    made = swap.install_groups(layer)
    assert made == [("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"), ("mlp.gate_proj", "mlp.up_proj")]
    a, m = layer.self_attn, layer.mlp
    counts = {"attn": _counting(a.q_proj._group), "mlp": _counting(m.gate_proj._group)}
    rng = np.random.default_rng(seed + 1)
    xb = O.f32_to_bf16_bits(rng.standard_normal((*lead, C)).astype(np.float32))
    x = bf16_tensor(xb, cuda)
    if xdt == "f32":
        x = x.float()
    dtype = x.dtype
    print(f"case shared-input {profile} x{tuple(x.shape)} {dtype}", flush=True)
    got = {n: getattr(a, n)(x) for n in ("q_proj", "k_proj", "v_proj")}
    got.update({n: getattr(m, n)(x) for n in ("gate_proj", "up_proj")})
    M = int(np.prod(lead))
    assert counts == {"attn": [M], "mlp": [M]}, "one launch per group"
    rows = x.reshape(-1, C)
    want_a = radix_ops.gemv_group([a.q_proj.p, a.k_proj.p, a.v_proj.p], rows, [qb, None, None], dtype)
    want_m = radix_ops.gemv_group([m.gate_proj.p, m.up_proj.p], rows, None, dtype)
    xf = O.bf16_bits_to_f32(xb).reshape(M, C)
    for n, w in zip(("q_proj", "k_proj", "v_proj", "gate_proj", "up_proj"), want_a + want_m):
        y = got[n]
        assert y.dtype == dtype and tuple(y.shape) == (*lead, w.shape[1]), n
        assert torch.equal(y.reshape(M, -1), w), f"{n}: not the grouped launch's rows"
        # the sums themselves: within the float64 bound (before the bias and the rounding)
        if n != "q_proj" and dtype == torch.float32:
            ref, bound = O.gemv_f64(bits[n], xf)
            err = np.abs(y.reshape(M, -1).cpu().numpy().astype(np.float64) - ref.reshape(M, -1)) / bound
            assert np.all(err <= 1.0), f"{n}: err/bound {err.max():.3f}"


def test_a_write_between_members_launches_again_and_dissolve_restores_single_launches(cuda):
    import torch

    from drinkme_amd import radix_ops, swap

    layer, bits, qb = _layer(cuda, "sip", 41)
    swap.install_groups(layer)
    a = layer.self_attn
    calls = _counting(a.q_proj._group)
    rng = np.random.default_rng(42)
    x = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal((1, C)).astype(np.float32)), cuda)
    ps = [a.q_proj.p, a.k_proj.p, a.v_proj.p]
    print("case shared-input write between members", flush=True)
    q = a.q_proj(x)
    before = radix_ops.gemv_group(ps, x, [qb, None, None], torch.bfloat16)
    x.mul_(-0.5)
    k, v = a.k_proj(x), a.v_proj(x)
    after = radix_ops.gemv_group(ps, x, [qb, None, None], torch.bfloat16)
    assert calls == [1, 1], "the write must launch the group again"
    assert torch.equal(q, before[0]) and torch.equal(k, after[1]) and torch.equal(v, after[2])
    a.q_proj._group.dissolve()
    for mod in (a.q_proj, a.k_proj, a.v_proj):
        assert torch.equal(mod(x), radix_ops.gemv_rows(mod.p, x, mod.bias, torch.bfloat16))
    assert calls == [1, 1]


@pytest.mark.parametrize("profile", ["sip", "gulp"])
def test_graph_of_member_calls_replays_the_grouped_launches(cuda, profile):
    """One capture of the members' calls (one grouped launch per group in
    the graph), replayed over new activations with eager work and
    synchronisations between the replays: every replay equals eager
    grouped launches on the same activation."""
    import torch

    from drinkme_amd import radix_ops, swap

    layer, bits, qb = _layer(cuda, profile, 7 if profile == "sip" else 8)
    swap.install_groups(layer)
    a, m = layer.self_attn, layer.mlp
    rng = np.random.default_rng(9)

    def fresh():
        return bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal((1, C)).astype(np.float32)), cuda)

    static_x = fresh()
    names = ("q_proj", "k_proj", "v_proj", "gate_proj", "up_proj")
    mods = [a.q_proj, a.k_proj, a.v_proj, m.gate_proj, m.up_proj]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the default stream, as torch asks before capture
        [mod(static_x) for mod in mods]
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print(f"case shared-input graph {profile}", flush=True)
    with torch.cuda.graph(graph):
        outs = [mod(static_x) for mod in mods]
    for rep in range(3):
        x = fresh()
        static_x.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        want = radix_ops.gemv_group([mod.p for mod in mods[:3]], x, [qb, None, None], torch.bfloat16)
        want += radix_ops.gemv_group([mod.p for mod in mods[3:]], x, None, torch.bfloat16)
        for n, o, w in zip(names, outs, want):
            assert torch.equal(o, w), f"replay {rep}: {n}"
        torch.cuda.synchronize()


def test_inference_mode_activations_share_the_launch(cuda):
    """Under torch.inference_mode (no version counter) the members match
    the activation by identity: one launch, the grouped launch's rows."""
    import torch

    from drinkme_amd import radix_ops, swap

    layer, bits, qb = _layer(cuda, "sip", 51)
    swap.install_groups(layer)
    a = layer.self_attn
    calls = _counting(a.q_proj._group)
    rng = np.random.default_rng(52)
    xb = O.f32_to_bf16_bits(rng.standard_normal((1, 1, C)).astype(np.float32))
    print("case shared-input inference mode", flush=True)
    with torch.inference_mode():
        x = bf16_tensor(xb, cuda).clone()
        assert x.is_inference()
        got = [a.q_proj(x), a.k_proj(x), a.v_proj(x)]
        want = radix_ops.gemv_group([a.q_proj.p, a.k_proj.p, a.v_proj.p], x.reshape(1, C), [qb, None, None],
                                    torch.bfloat16)
    assert calls == [1]
    for g, w in zip(got, want):
        assert torch.equal(g.reshape(1, -1), w)
