"""GPU parity over seeded random launches: profile (sip, gulp), a group of 1
to 4 tensors sharing x, row counts from 1 to 12288, columns from 1024 to
25600 (whole blocks, so the fast kernels take them), M = 1..8, and three
exponent distributions (tight, spread, escape-heavy). Every output must lie
within the float64 bound of the oracle's dot over the source bits, as in
the fixed-shape tests; this sweep reaches tile heights, tensor boundaries
inside tiles, column phases and progress-balanced launches that those
shapes do not pick out one by one."""

import numpy as np
import pytest

from oracle import radix_oracle as O
from tests.helpers import bf16_tensor, escape_heavy_bits, finite_bits, oracle_dict

pytestmark = pytest.mark.gpu

CASES = 16


def _case(k):
    rng = np.random.default_rng(90210 + k)
    prof = str(rng.choice(["sip", "gulp"]))
    n = int(rng.integers(1, 5))
    C = int(rng.choice([1024, 2048, 3072, 4096, 5120, 8192, 12288, 16384, 25600]))
    M = int(rng.integers(1, 9))
    rows = [int(rng.integers(1, 3000)) if rng.random() < 0.7 else int(rng.choice([1024, 4096, 6144, 12288]))
            for _ in range(n)]
    while sum(rows) * C > 40_000_000:
        rows = [max(1, r // 2) for r in rows]
    kind = str(rng.choice(["tight", "spread", "escapes"]))
    return rng, prof, rows, C, M, kind


@pytest.mark.parametrize("k", range(CASES))
def test_random_launch_matches_the_oracle(cuda, k):
    import torch

    from drinkme_amd import radix_ops, swap

    rng, prof, rows, C, M, kind = _case(k)
    bits = [escape_heavy_bits(rng, (r, C), 0.05) if kind == "escapes" else finite_bits(rng, (r, C), spread=kind == "spread")
            for r in rows]
    rts = [swap.to_device_radix(oracle_dict(b, prof), cuda) for b in bits]
    xb = O.f32_to_bf16_bits(rng.standard_normal((M, C)).astype(np.float32))
    x = bf16_tensor(xb, cuda)
    xf = O.bf16_bits_to_f32(xb)
    print(f"case {k}: {prof} rows={rows} C={C} M={M} {kind}", flush=True)
    ys = radix_ops.gemv_group(rts, x, None, torch.float32)
    for i, (y, b) in enumerate(zip(ys, bits)):
        ref, bound = O.gemv_f64(b, xf)
        err = np.abs(y.cpu().numpy().astype(np.float64).reshape(ref.shape) - ref) / bound
        assert np.all(err <= 1.0), f"case {k} tensor {i}: err/bound {err.max():.3f}"
