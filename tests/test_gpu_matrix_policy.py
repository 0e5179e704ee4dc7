"""GPU parity under the matrix policy (dmx_radix_set_policy(DMX_POLICY_MATRIX),
radix_ops.set_policy("matrix")): gulp's 3- and 4-row verify in quad units on
the matrix cores, as 8 rows run under either policy.

  - every output within the float64 bound of the oracle's dot over the
    source bits, with the bias epilogue exact, through the single and the
    grouped launch, on rows long enough for column phases;
  - the raw twin follows the policy: under it, the twin equals its
    compressed tensor bit for bit, as under AUTO;
  - the policy is process-global: every test restores the one it found.
"""

import contextlib
import zlib

import numpy as np
import pytest

from oracle import radix_oracle as O
from tests.helpers import bf16_tensor, escape_heavy_bits, finite_bits, oracle_dict

pytestmark = pytest.mark.gpu


@contextlib.contextmanager
def _policy(name):
    from drinkme_amd import radix_ops

    prev = radix_ops.set_policy(name)
    try:
        yield
    finally:
        radix_ops.set_policy(prev)


def _check(y, xf, bits, what):
    ref, bound = O.gemv_f64(bits, xf)
    err = np.abs(np.asarray(y, np.float64).reshape(ref.shape) - ref) / bound
    assert np.all(err <= 1.0), f"{what}: err/bound {err.max():.3f}"


@pytest.mark.parametrize("shape", [(512, 4096), (1000, 2048), (64, 24576), (3, 1024)])
@pytest.mark.parametrize("M", [3, 4])
def test_gulp_verify_rows_on_the_matrix_cores_match_the_oracle(cuda, shape, M):
    import torch

    from drinkme_amd import radix_ops, swap

    R, C = shape
    rng = np.random.default_rng(zlib.crc32(repr(("matrix", shape, M)).encode()))
    bits = escape_heavy_bits(rng, shape, 0.05) if R == 1000 else finite_bits(rng, shape, spread=True)
    p = swap.to_device_radix(oracle_dict(bits, "gulp"), cuda)
    xb = O.f32_to_bf16_bits(rng.standard_normal((M, C)).astype(np.float32))
    x = bf16_tensor(xb, cuda)
    xf = O.bf16_bits_to_f32(xb)
    bias = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal(R).astype(np.float32)), cuda)
    print(f"case matrix policy gulp {shape} M={M}", flush=True)
    with _policy("matrix"):
        y = radix_ops.gemv_mc(p, x)
        fused = radix_ops.gemv_rows(p, x, bias, torch.bfloat16)
        again = radix_ops.gemv_mc(p, x)
    _check(y.cpu().numpy(), xf, bits, f"matrix {shape} M={M}")
    assert torch.equal(fused, (y + bias.float()).to(torch.bfloat16)), "the bias epilogue"
    assert torch.equal(again, y), "deterministic"
    with _policy("auto"):
        y_auto = radix_ops.gemv_mc(p, x)
    _check(y_auto.cpu().numpy(), xf, bits, f"auto {shape} M={M}")


@pytest.mark.parametrize("rows,C", [((4096, 1024, 1024), 4096), ((12288, 12288), 4096), ((640, 128, 128), 1024)])
def test_gulp_groups_under_the_matrix_policy_match_the_oracle(cuda, rows, C):
    import torch

    from drinkme_amd import radix_ops, swap

    rng = np.random.default_rng(zlib.crc32(repr(("matrix group", rows, C)).encode()))
    bits = [finite_bits(rng, (r, C), spread=i % 2 == 1) for i, r in enumerate(rows)]
    rts = [swap.to_device_radix(oracle_dict(b, "gulp"), cuda) for b in bits]
    xb = O.f32_to_bf16_bits(rng.standard_normal((4, C)).astype(np.float32))
    x = bf16_tensor(xb, cuda)
    xf = O.bf16_bits_to_f32(xb)
    print(f"case matrix policy gulp group rows={rows} C={C}", flush=True)
    with _policy("matrix"):
        ys = radix_ops.gemv_group(rts, x, None, torch.float32)
    for i, (y, b) in enumerate(zip(ys, bits)):
        _check(y.cpu().numpy(), xf, b, f"matrix group {rows} tensor {i}")


@pytest.mark.parametrize("shape", [(512, 4096), (300, 8192), (1000, 2048)])
def test_the_twin_follows_the_matrix_policy_bit_for_bit(cuda, shape):
    import torch

    from drinkme_amd import radix_ops, swap

    R, C = shape
    rng = np.random.default_rng(zlib.crc32(repr(("matrix twin", shape)).encode()))
    bits = finite_bits(rng, shape, spread=True)
    p = swap.to_device_radix(oracle_dict(bits, "gulp"), cuda)
    twin = swap.to_device_twin(bf16_tensor(bits, cuda), widths=p["widths"], device=cuda)
    xb = O.f32_to_bf16_bits(rng.standard_normal((4, C)).astype(np.float32))
    x = bf16_tensor(xb, cuda)
    bias = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal(R).astype(np.float32)), cuda)
    print(f"case matrix policy twin {shape}", flush=True)
    with _policy("matrix"):
        for M in (3, 4):
            a, b = radix_ops.gemv_mc(twin, x[:M]), radix_ops.gemv_mc(p, x[:M])
            assert torch.equal(a, b), f"M={M}: max |diff| {(a - b).abs().max().item():.3g}"
        assert torch.equal(radix_ops.gemv_rows(twin, x, bias, torch.bfloat16),
                           radix_ops.gemv_rows(p, x, bias, torch.bfloat16)), "fused bias"
    _check(a.cpu().numpy(), O.bf16_bits_to_f32(xb), bits, f"twin {shape}")


def test_the_policy_switch_reports_and_restores(cuda):
    from drinkme_amd import radix_ops

    prev = radix_ops.set_policy("matrix")
    try:
        assert radix_ops.set_policy("generic") == "matrix"
        assert radix_ops.set_policy("matrix") == "generic"
    finally:
        assert radix_ops.set_policy(prev) == "matrix"
