"""GPU parity at the full sizes of the measured workloads, through the
grouped launch path the benchmark times (dmx_radix_gemv_group: q/k/v and
gate/up of a layer as one launch each, o and down alone).

  - the single 4096 x 4096 linear, N(0, 0.02), sip, M = 1;
  - Qwen3-8B layer (4096 hidden; q 4096x4096, k/v 1024x4096, o 4096x4096,
    gate/up 12288x4096, down 4096x12288), N(0, 0.02), sip, M = 1;
  - the same layer at gulp, M = 4 (the MTP verify rows), also under the
    matrix policy (gulp's verify rows in quad units on the matrix cores),
    and at sip, M = 4 (its blocks contracted on the matrix cores);
  - the Qwen3-8B lm_head, 151936 x 4096 N(0, 0.02), sip, M = 1: the largest
    launch of the decode-step sweep, with its own plan (about 2,400 blocks
    per CU, progress balance on);
  - the 32B-class layer (hidden 5120; q 8192x5120, k/v 1024x5120, o
    5120x8192, gate/up 25600x5120, down 5120x25600), Student-t(4) weights
    scaled to std 0.02, gulp at M = 1 and M = 4 (the down projection at
    M = 4 runs in column phases), and sip at M = 1.

The weights are the benchmark's own streams (drinkme_amd.synth), packed by
the product encoder as bench.py packs them. Bars, as drinkme's gates put
them (bench/radix_gemv_bitpin.py:181-191, bench/radix_mc_bitpin.py:81-116):
  - the decoded bits equal the source bits, every weight;
  - every output column of every row within the float64 bound
    2e-6 |x|.|W| + 1e-7 of the oracle's dot over the source bits;
  - the bf16 output equal to the fp32 output rounded once (same launch
    plan, same sums), and within 1e-2 relative of decode-then-matmul
    (fp32 accumulate, bf16 out).
"""

import time

import numpy as np
import pytest

from oracle import radix_oracle as O
from tests.helpers import bf16_tensor, gemv_f32_rows, gemv_f64_rows, planted_mistakes_rejected

pytestmark = pytest.mark.gpu

REL_TOL = 1e-2  # relative tolerance of the bf16 output vs decode-then-matmul
GROUPS = (("q", "k", "v"), ("o",), ("gate", "up"), ("down",))


def _log(t0, msg):
    print(f"[{time.time() - t0:6.1f} s] {msg}", flush=True)


def _resident(bits, profile, device):
    from drinkme_amd import radix_pack, swap

    p = radix_pack.pack_array_radix(bits, profile)
    assert p is not None, "the tensor must ride the compressed streams"
    return swap.to_device_radix(p, device)


def _check_group(cuda, t0, what, tensors, x_bits):
    """tensors: [(name, source bits, runtime dict)] sharing x_bits [M, C]."""
    import torch

    from drinkme_amd import radix_ops

    for name, bits, rt in tensors:
        got = radix_ops.decode_bits(rt).view(torch.int16)
        want = torch.from_numpy(bits.view(np.int16)).to(cuda)
        assert torch.equal(got, want), f"{what} {name}: decoded bits differ from the source"
        del got, want
    x = bf16_tensor(x_bits, cuda)
    xf = O.bf16_bits_to_f32(x_bits)
    rts = [rt for _, _, rt in tensors]
    y32 = radix_ops.gemv_group(rts, x, None, torch.float32)
    yb = radix_ops.gemv_group(rts, x, None, torch.bfloat16)
    torch.cuda.synchronize()
    for (name, bits, _), a, b in zip(tensors, y32, yb):
        assert torch.equal(b, a.to(torch.bfloat16)), f"{what} {name}: bf16 output is not the fp32 output rounded once"
        ref, bound = gemv_f64_rows(bits, xf)
        got = a.cpu().numpy().astype(np.float64)
        err = np.abs(got - ref) / bound
        assert np.all(err <= 1.0), f"{what} {name}: err/bound {err.max():.3f} at {np.unravel_index(err.argmax(), err.shape)}"
        # the check is not unfailable: three mistakes planted in the oracle
        # at the row this launch came closest on must each be rejected
        m, r = np.unravel_index(err.argmax(), err.shape)
        planted = planted_mistakes_rejected(got[m], bits, xf[m], int(r))
        assert planted is not None and min(planted) > 1.0, f"{what} {name}: a planted mistake passed ({planted})"
        ref32 = gemv_f32_rows(bits, xf)
        want_bf16 = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref32)).astype(np.float64)
        gotb = b.float().cpu().numpy().astype(np.float64)
        # relative to the value, floored at 1e-3 of the row's |x|.|W| (a sum
        # that cancels to near zero has no relative digits to compare)
        scale = np.maximum(np.abs(want_bf16), (bound - 1e-7) / 2e-6 * 1e-3)
        assert np.all(np.abs(gotb - want_bf16) <= REL_TOL * scale), f"{what} {name}: 1e-2 relative"
        _log(t0, f"{what} {name} {bits.shape}: bits exact, max err/bound {err.max():.3f}")


def _layer(cuda, workload, copy, shapes, dist, profile, m, x_workload):
    from drinkme_amd import synth

    t0 = time.time()
    print(f"case full layer {workload} {profile} M={m}", flush=True)
    rows = {n: (r, c) for n, r, c in shapes}
    for grp in GROUPS:
        C = rows[grp[0]][1]
        tensors = []
        for name in grp:
            R = rows[name][0]
            bits = synth.weight(workload, copy, name, R, C, dist)
            tensors.append((name, bits, _resident(bits, profile, cuda)))
        _log(t0, f"packed {'/'.join(grp)}")
        xb = synth.activation(x_workload, f"x{C}", m, C)
        _check_group(cuda, t0, f"{workload} {profile} M={m}", tensors, xb)
        del tensors
        import torch

        torch.cuda.empty_cache()


def test_linear_4096_sip_m1(cuda):
    """The single-linear workload's first copy, the bench's own tensor."""
    from drinkme_amd import synth

    t0 = time.time()
    print("case linear 4096x4096 sip M=1", flush=True)
    bits = synth.weight("linear-4096", 0, "w", 4096, 4096)
    rt = _resident(bits, "sip", cuda)
    xb = synth.activation("linear-4096", "x4096", 1, 4096)
    _check_group(cuda, t0, "linear-4096 sip M=1", [("w", bits, rt)], xb)


def test_qwen3_8b_layer_sip_m1(cuda):
    from drinkme_amd import synth

    _layer(cuda, "qwen3-8b", 0, synth.QWEN3_8B_LAYER, synth.NORMAL, "sip", 1, "qwen3-8b-step")


def test_qwen3_8b_layer_gulp_m4(cuda):
    from drinkme_amd import synth

    _layer(cuda, "qwen3-8b", 0, synth.QWEN3_8B_LAYER, synth.NORMAL, "gulp", 4, "qwen3-8b-layer")


def test_qwen3_8b_layer_gulp_m4_matrix_cores(cuda):
    """The same C3 layer under the matrix policy: gulp's four verify rows in
    quad units on the matrix cores (AUTO keeps them on v_dot2)."""
    from drinkme_amd import radix_ops, synth

    prev = radix_ops.set_policy("matrix")
    try:
        _layer(cuda, "qwen3-8b", 0, synth.QWEN3_8B_LAYER, synth.NORMAL, "gulp", 4, "qwen3-8b-layer")
    finally:
        radix_ops.set_policy(prev)


def test_qwen3_8b_layer_sip_m4(cuda):
    from drinkme_amd import synth

    _layer(cuda, "qwen3-8b", 0, synth.QWEN3_8B_LAYER, synth.NORMAL, "sip", 4, "qwen3-8b-layer")


def test_qwen3_8b_lm_head_sip_m1(cuda):
    """The decode-step sweep's lm_head launch, the bench's own tensor."""
    from drinkme_amd import synth

    t0 = time.time()
    name, R, C = synth.QWEN3_8B_LM_HEAD
    print(f"case lm_head {R}x{C} sip M=1", flush=True)
    bits = synth.weight("qwen3-8b", "head", name, R, C)
    rt = _resident(bits, "sip", cuda)
    _log(t0, "packed lm_head")
    xb = synth.activation("qwen3-8b-step", f"x{C}", 1, C)
    _check_group(cuda, t0, "qwen3-8b sip M=1", [(name, bits, rt)], xb)


@pytest.mark.parametrize("m", [1, 4])
def test_32b_layer_gulp_student_t(cuda, m):
    from drinkme_amd import synth

    _layer(cuda, "32b-class", 0, synth.CLASS_32B_LAYER, synth.STUDENT_T4, "gulp", m, "32b-layer")


def test_32b_layer_sip_student_t_m1(cuda):
    from drinkme_amd import synth

    _layer(cuda, "32b-class", 0, synth.CLASS_32B_LAYER, synth.STUDENT_T4, "sip", 1, "32b-layer")
