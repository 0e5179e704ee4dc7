"""GPU parity: the fused decode + GEMV (dmx_radix_gemv) against the oracle,
through the C ABI.

Bars (drinkme's bench/radix_gemv_bitpin.py:181-191, bench/radix_mc_bitpin.py,
tests/test_codec_bias_rounding.py, and the north star's 1e-2):
  - fp32 GEMV within the float64 bound 2e-6 |x|.|W| + 1e-7 of the oracle's
    float64 dot over the source bits;
  - the fused bf16 output with bias == (fp32 result + bias) rounded once;
  - every column of an M = 2..8 call within the same bound;
  - bf16 outputs within 1e-2 relative of decode-then-matmul (fp32
    accumulate, bf16 out);
  - the bias cancellation known answer 0.00390625 on every arm.
"""

import zlib

import numpy as np
import pytest

from oracle import radix_oracle as O
from tests.helpers import bf16_tensor, escape_heavy_bits, finite_bits, oracle_dict, u16_of

pytestmark = pytest.mark.gpu

PROFILES = ("sip", "balanced", "gulp")
BOUND_TOL = 1.0  # |y - y64| <= bound, the float64 oracle's cancellation-aware bound
REL_TOL = 1e-2   # the north star's relative tolerance vs decode-then-matmul


def _check_bound(y, x_f32, bits, what):
    ref, bound = O.gemv_f64(bits, x_f32)
    err = np.abs(np.asarray(y, np.float64) - ref) / bound
    assert np.all(err <= BOUND_TOL), f"{what}: err/bound {err.max():.3f}"
    return ref


def _run_shape(cuda, bits, profile, rng, ms=(1, 3, 8), stored_raw=False):
    import torch

    from drinkme_amd import radix_ops, swap

    R, C = bits.shape
    if stored_raw:
        # the tensor drinkme stores raw (radix would expand it): served from
        # its raw bits, here through the twin of the profile's widths
        rt = swap.to_device_twin(bf16_tensor(bits, cuda), widths=O.PROFILES[profile], device=cuda)
    else:
        rt = swap.to_device_radix(oracle_dict(bits, profile), cuda)
    bias_bits = O.f32_to_bf16_bits(np.linspace(-0.1, 0.1, R).astype(np.float32))
    bias = bf16_tensor(bias_bits, cuda)
    for M in ms:
        xb = O.f32_to_bf16_bits(rng.standard_normal((M, C)).astype(np.float32))
        x = bf16_tensor(xb, cuda)
        xf = O.bf16_bits_to_f32(xb)
        y32 = radix_ops.gemv_rows(rt, x, None, torch.float32).cpu().numpy()
        _check_bound(y32, xf, bits, f"{profile} {bits.shape} M={M} bf16 x")
        fused = radix_ops.gemv_rows(rt, x, bias, torch.bfloat16)
        want = (torch.from_numpy(y32).to(cuda) + bias.float()).to(torch.bfloat16)
        assert torch.equal(fused, want), f"{profile} {bits.shape} M={M}: fused epilogue"
        # fp32 activations take the widened path
        x32 = torch.from_numpy(rng.standard_normal((M, C)).astype(np.float32)).to(cuda)
        y = radix_ops.gemv_rows(rt, x32, None, torch.float32).cpu().numpy()
        _check_bound(y, x32.cpu().numpy(), bits, f"{profile} {bits.shape} M={M} fp32 x")
        # decode-then-matmul: fp32 accumulate over the oracle's decoded weight, bf16 out
        ref32 = O.gemv_f32(bits, xf, O.bf16_bits_to_f32(bias_bits))
        got = fused.float().cpu().numpy()
        want_bf16 = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref32))
        scale = np.maximum(np.abs(want_bf16), np.abs(xf) @ np.abs(O.bf16_bits_to_f32(bits)).T * 1e-3 + 1e-6)
        assert np.all(np.abs(got - want_bf16) <= REL_TOL * scale), f"{profile} {bits.shape} M={M}: 1e-2 relative"


@pytest.mark.parametrize("shape", [(1, 1), (7, 33), (3, 1025), (129, 260), (17, 3079)])
@pytest.mark.parametrize("spread", [False, True])
@pytest.mark.parametrize("profile", PROFILES)
def test_ragged_shapes(cuda, shape, spread, profile):
    rng = np.random.default_rng(zlib.crc32(repr((shape, spread, profile)).encode()))
    bits = finite_bits(rng, shape, spread)
    raw = O.pack(bits, profile).raw  # (1, 1): radix would expand it, so it is stored raw
    print(f"case gemv ragged {shape} spread={spread} {profile} raw={raw}", flush=True)
    _run_shape(cuda, bits, profile, rng, stored_raw=raw)


@pytest.mark.parametrize("shape", [(1024, 4096), (256, 12288), (4096, 1024)])
@pytest.mark.parametrize("profile", PROFILES)
def test_production_shapes(cuda, shape, profile):
    rng = np.random.default_rng(zlib.crc32(repr((shape, profile)).encode()))
    bits = finite_bits(rng, shape, spread=True)
    print(f"case gemv production {shape} {profile}", flush=True)
    _run_shape(cuda, bits, profile, rng, ms=(1, 4))


@pytest.mark.parametrize("rate", [0.0, 0.02, 0.1, 0.45])
def test_sip_fast_path_escape_rates(cuda, rate):
    """The sip M = 1 kernel across escape densities: none, typical, and a
    terminal longer than 64 words (> 256 escapes per block)."""
    import torch

    from drinkme_amd import radix_ops, swap

    rng = np.random.default_rng(int(rate * 1000) + 7)
    bits = escape_heavy_bits(rng, (512, 4096), rate)
    d = oracle_dict(bits, "sip")
    rt = swap.to_device_radix(d, cuda)
    xb = O.f32_to_bf16_bits(rng.standard_normal((1, 4096)).astype(np.float32))
    x = bf16_tensor(xb, cuda)
    print(f"case sip escapes rate={rate}", flush=True)
    y = radix_ops.gemv(rt, x[0]).cpu().numpy()
    _check_bound(y[None], O.bf16_bits_to_f32(xb), bits, f"sip escapes {rate}")
    prev = radix_ops.set_policy("generic")
    try:
        yg = radix_ops.gemv(rt, x[0]).cpu().numpy()
    finally:
        radix_ops.set_policy(prev)
    _check_bound(yg[None], O.bf16_bits_to_f32(xb), bits, f"sip escapes {rate} generic")
    assert torch.cuda.is_available()


def test_sip_4096_square(cuda):
    """The single-linear workload: 4096 x 4096 N(0, 0.02) at sip, x N(0, 1)."""
    import torch

    from drinkme_amd import radix_ops, radix_pack, swap, synth

    bits = synth.weight("c1", 0, "w", 4096, 4096)
    p = radix_pack.pack_array_radix(bits, "sip")
    rt = swap.to_device_radix(p, cuda)
    assert np.array_equal(u16_of(radix_ops.decode_bits(rt)), bits)
    xb = synth.activation("c1", "x", 1, 4096)
    x = bf16_tensor(xb, cuda)
    y = radix_ops.gemv(rt, x[0]).cpu().numpy()
    _check_bound(y[None], O.bf16_bits_to_f32(xb), bits, "c1")
    fused = radix_ops.gemv_fused(rt, x[0], None, torch.bfloat16).float().cpu().numpy()
    ref32 = O.gemv_f32(bits, O.bf16_bits_to_f32(xb))
    want = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref32))
    rel = np.abs(fused - want) / np.maximum(np.abs(want), 1e-3)
    assert np.median(rel) < 1e-2 and np.all(np.abs(fused - want) <= 1e-2 * np.maximum(np.abs(want), 0.05))


@pytest.mark.parametrize("profile", PROFILES)
@pytest.mark.parametrize("rows", [1, 4])
def test_bias_rounds_once(cuda, profile, rows):
    """W columns 0, 1 = 1, x = [1, 1/256, 0 ...], bias = -1: the fp32
    accumulator 1.00390625 minus 1 is 2^-8; rounding first would give 0
    (tests/test_codec_bias_rounding.py:1-19)."""
    import torch

    from drinkme_amd import swap

    R = C = 1024
    w = np.zeros((R, C), np.float32)
    w[:, :2] = 1
    bits = O.f32_to_bf16_bits(w)
    d = oracle_dict(bits, profile)
    mod = swap.make_module(d, torch.full((R,), -1.0, dtype=torch.bfloat16, device=cuda), cuda)
    x = torch.zeros(rows, C, dtype=torch.bfloat16, device=cuda)
    x[:, 0] = 1
    x[:, 1] = 1 / 256
    assert mod._route(x) == ("gemv" if rows == 1 else "mc")
    out = mod(x)
    assert torch.all(out == 0.00390625), out.flatten()[:4]


@pytest.mark.parametrize("R", [1, 3, 17, 100, 1000, 5000])
@pytest.mark.parametrize("C", [1024, 2048, 5120, 12288])
def test_sip_work_split(cuda, R, C):
    """The sip kernel's row tiles and segments over awkward row counts and
    every column-block count the workloads use (1, 2, 5, 12 blocks)."""
    import torch

    from drinkme_amd import radix_ops, swap

    rng = np.random.default_rng(R * 100003 + C)
    bits = escape_heavy_bits(rng, (R, C), 0.03)
    d = oracle_dict(bits, "sip")
    rt = swap.to_device_radix(d, cuda)
    xb = O.f32_to_bf16_bits(rng.standard_normal((1, C)).astype(np.float32))
    x = bf16_tensor(xb, cuda)
    bias_bits = O.f32_to_bf16_bits(rng.standard_normal(R).astype(np.float32))
    print(f"case sip split R={R} C={C}", flush=True)
    y = radix_ops.gemv(rt, x[0]).cpu().numpy()
    _check_bound(y[None], O.bf16_bits_to_f32(xb), bits, f"sip split {R}x{C}")
    fused = radix_ops.gemv_fused(rt, x[0], bf16_tensor(bias_bits, cuda), torch.bfloat16)
    want = (torch.from_numpy(y).to(cuda) + bf16_tensor(bias_bits, cuda).float()).to(torch.bfloat16)
    assert torch.equal(fused.reshape(-1), want)


def _gulp_bits(rng, kind, shape):
    from drinkme_amd import synth

    R, C = shape
    if kind == "normal":
        return synth.weight("gulp-test", 0, "w", R, C)
    if kind == "t4":
        return synth.weight("gulp-test", 0, "t4", R, C, synth.STUDENT_T4)
    if kind == "spread":
        return finite_bits(rng, shape, spread=True)
    if kind == "long-tail":
        # the ordinary rows set the palette (90% on three exponents, 6% on
        # three more, 4% over 15 rare ones); every third row's blocks hold
        # 68% tier-1 exponents and 1% past the palette: tails (tier 1, tier 2
        # and the terminal) of 65-75 words, past the one word a lane loads,
        # most with at most 128 tier-1 escapes (so only the tail's length
        # sends them down the exact path)
        u = rng.random(shape)
        exps = np.where(u < 0.9, rng.integers(120, 123, size=shape),
                        np.where(u < 0.96, rng.integers(116, 119, size=shape), rng.integers(60, 75, size=shape)))
        rows = np.arange(R) % 3 == 0
        v = rng.random((int(rows.sum()), C))
        exps[rows] = np.where(v < 0.2, rng.integers(120, 123, size=v.shape),
                              np.where(v < 0.88, rng.integers(116, 119, size=v.shape),
                                       np.where(v < 0.99, rng.integers(60, 75, size=v.shape),
                                                rng.integers(20, 40, size=v.shape))))
        exps = exps.astype(np.uint16)
    elif kind == "dense-tier1":
        # 12 equally likely exponents: half the weights escape tier 1 (more
        # than 128 per block: the lane-serial path)
        exps = rng.integers(100, 112, size=shape).astype(np.uint16)
    elif kind == "terminal":
        # 90% on three exponents, 5% on three more, 5% over 40 rare ones:
        # about 50 tier-1 escapes per block (the windowed path), 25 of the
        # rare exponents past tier 2 (about 3% of the weights in the terminal)
        u = rng.random(shape)
        exps = np.where(u < 0.9, rng.integers(120, 123, size=shape),
                        np.where(u < 0.95, rng.integers(116, 119, size=shape),
                                 rng.integers(60, 100, size=shape))).astype(np.uint16)
    else:
        # 70% on three exponents, 30% over 40 rare ones: about 280 tier-1
        # escapes per block (the lane-serial path), 16% of the weights in
        # the terminal
        exps = np.where(rng.random(shape) < 0.7, rng.integers(120, 123, size=shape),
                        rng.integers(60, 100, size=shape)).astype(np.uint16)
    bits = (exps << 7) | rng.integers(0, 128, shape, dtype=np.uint16)
    return bits | (rng.integers(0, 2, shape, dtype=np.uint16) << 15)


@pytest.mark.parametrize("kind", ["normal", "t4", "spread", "terminal", "dense-tier1", "terminal-heavy", "long-tail"])
@pytest.mark.parametrize("M", [1, 3, 8])
def test_gulp_fast_path(cuda, kind, M):
    """The gulp kernel (M = 1..8) across tier-1, tier-2 and terminal escape
    densities, against the float64 bound and the generic kernel; with and
    without the schedule in the descriptor."""
    import torch

    from drinkme_amd import radix_ops, swap

    rng = np.random.default_rng(zlib.crc32(repr((kind, M)).encode()))
    shape = (300, 3072)
    bits = _gulp_bits(rng, kind, shape)
    pk = O.pack(bits, "gulp")
    if pk.raw:
        pytest.skip("stored raw")
    if kind == "long-tail":
        tail = np.diff(pk.offsets.astype(np.int64)) - 320
        assert ((tail > 64) & ((O.schedule(pk) >> 8) <= 16)).sum() > 100, "the case lost its long tails"
    rt = swap.to_device_radix(oracle_dict(bits, "gulp"), cuda)
    xb = O.f32_to_bf16_bits(rng.standard_normal((M, shape[1])).astype(np.float32))
    x = bf16_tensor(xb, cuda)
    print(f"case gulp fast {kind} M={M}", flush=True)
    y = radix_ops.gemv_rows(rt, x, None, torch.float32).cpu().numpy()
    _check_bound(y, O.bf16_bits_to_f32(xb), bits, f"gulp {kind} M={M}")
    # the kernel finds its streams from each block's counts, not the
    # schedule: a descriptor without one runs the same kernel, bit for bit
    bare = dict(rt, rx_schedule=torch.empty(0, dtype=torch.uint16, device=cuda))
    assert np.array_equal(radix_ops.gemv_rows(bare, x, None, torch.float32).cpu().numpy(), y), "without schedule"
    bias = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal(shape[0]).astype(np.float32)), cuda)
    fused = radix_ops.gemv_rows(rt, x, bias, torch.bfloat16)
    assert torch.equal(fused, (torch.from_numpy(y).to(cuda) + bias.float()).to(torch.bfloat16))
    prev = radix_ops.set_policy("generic")
    try:
        yg = radix_ops.gemv_rows(rt, x, None, torch.float32).cpu().numpy()
    finally:
        radix_ops.set_policy(prev)
    _check_bound(yg, O.bf16_bits_to_f32(xb), bits, f"gulp {kind} M={M} generic")


def test_threads_with_different_lds_needs(cuda):
    """Launches from several host threads (a stream each) whose plans need
    different dynamic-LDS limits: every call succeeds and equals the
    single-threaded result bit for bit (the limit only ever rises)."""
    import threading

    import torch

    from drinkme_amd import radix_ops, swap

    rng = np.random.default_rng(31)
    shapes = [(256, 2048), (128, 16384), (256, 32768)]
    rts, xs, want = [], [], []
    for R, C in shapes:
        bits = finite_bits(rng, (R, C))
        rt = swap.to_device_radix(oracle_dict(bits, "sip"), cuda)
        x = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal((8, C)).astype(np.float32)), cuda)
        rts.append(rt)
        xs.append(x)
    for rt, x in zip(rts, xs):
        want.append([radix_ops.gemv_mc(rt, x[:m]) for m in (2, 4, 8)])
    torch.cuda.synchronize()
    errors = []

    def worker(k):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for it in range(6):
                    i = (k + it) % len(shapes)
                    for j, m in enumerate((2, 4, 8)):
                        got = radix_ops.gemv_mc(rts[i], xs[i][:m])
                        s.synchronize()
                        if not torch.equal(got, want[i][j]):
                            errors.append(f"thread {k} shape {shapes[i]} M={m}")
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(f"thread {k}: {e}")

    print("case threads lds", flush=True)
    ts = [threading.Thread(target=worker, args=(k,)) for k in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors
