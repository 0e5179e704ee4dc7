"""GPU: the raw twin (dmx_radix_gemv_twin) against its compressed tensor,
bit for bit — drinkme's order-matched twin claim (bench/radix_twin_bitpin.py:
1-40; swap.to_device_twin src/drinkme/codec/swap.py:169-198): the twin runs
the kernel the compressed tensor of its widths runs, with the decode
replaced by a load of the raw weight at the same (row, column), so at any
one launch plan the two outputs are identical.

Covered: every profile (sip and gulp on their fast kernels, balanced on the
generic one), M = 1..8, fp32 and bf16 outputs, the fused bias epilogue, a
row long enough for column phases at M = 8, columns that are not a whole
number of blocks (the generic kernel at every profile), an fp32
activation (the generic kernel's widening path), and a 12288 x 4096
launch long enough for the sip kernel's progress balance.
"""

import zlib

import numpy as np
import pytest

from oracle import radix_oracle as O
from tests.helpers import bf16_tensor, escape_heavy_bits, finite_bits, oracle_dict

pytestmark = pytest.mark.gpu


def _pair(bits, profile, cuda):
    from drinkme_amd import swap

    p = swap.to_device_radix(oracle_dict(bits, profile), cuda)
    twin = swap.to_device_twin(bf16_tensor(bits, cuda), widths=p["widths"], device=cuda)
    return p, twin


@pytest.mark.parametrize("profile", ["sip", "gulp", "balanced"])
@pytest.mark.parametrize("shape", [(512, 4096), (300, 3584), (1000, 2048)])
def test_twin_is_its_compressed_tensor_bit_for_bit(cuda, profile, shape):
    import torch

    from drinkme_amd import radix_ops

    rng = np.random.default_rng(zlib.crc32(repr(("twin", profile, shape)).encode()))
    R, C = shape
    bits = escape_heavy_bits(rng, shape, 0.03) if R == 1000 else finite_bits(rng, shape, spread=True)
    p, twin = _pair(bits, profile, cuda)
    xb = O.f32_to_bf16_bits(rng.standard_normal((8, C)).astype(np.float32))
    x = bf16_tensor(xb, cuda)
    bias = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal(R).astype(np.float32)), cuda)
    print(f"case twin {profile} {shape}", flush=True)
    assert torch.equal(radix_ops.gemv(twin, x[0]), radix_ops.gemv(p, x[0])), "gemv M=1"
    assert torch.equal(radix_ops.gemv_fused(twin, x[0], bias), radix_ops.gemv_fused(p, x[0], bias)), "fused"
    for M in range(2, 9):
        a, b = radix_ops.gemv_mc(twin, x[:M]), radix_ops.gemv_mc(p, x[:M])
        assert torch.equal(a, b), f"gemv_mc M={M}: max |diff| {(a - b).abs().max().item():.3g}"
    # an fp32 activation: both run the generic kernel
    xf = x[:3].float()
    assert torch.equal(radix_ops.gemv_mc(twin, xf), radix_ops.gemv_mc(p, xf)), "fp32 x"
    # and the twin is right, not only equal
    ref, bound = O.gemv_f64(bits, O.bf16_bits_to_f32(xb[:1]))
    y = radix_ops.gemv(twin, x[0]).cpu().numpy().astype(np.float64)
    assert np.all(np.abs(y - ref.reshape(y.shape)) <= bound.reshape(y.shape))


@pytest.mark.parametrize("profile", ["sip", "gulp"])
def test_twin_matches_through_column_phases(cuda, profile):
    """M = 8 over 16384 columns needs 256 KB of activation rows: the fast
    kernels run it in column phases, and the twin in the same phases."""
    import torch

    from drinkme_amd import radix_ops

    rng = np.random.default_rng(91 + len(profile))
    R, C = 128, 16384
    bits = finite_bits(rng, (R, C), spread=True)
    p, twin = _pair(bits, profile, cuda)
    x = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal((8, C)).astype(np.float32)), cuda)
    print(f"case twin phases {profile}", flush=True)
    for M in (1, 4, 8):
        assert torch.equal(radix_ops.gemv_mc(twin, x[:M]) if M > 1 else radix_ops.gemv(twin, x[0]),
                           radix_ops.gemv_mc(p, x[:M]) if M > 1 else radix_ops.gemv(p, x[0])), f"M={M}"


def test_plain_linear_twin_takes_sips_kernel(cuda):
    """A stock Linear's twin (raw_gemv_dict: sip's widths) is the sip
    kernel's order: bit for bit the sip-packed tensor."""
    import torch

    from drinkme_amd import radix_ops, swap

    rng = np.random.default_rng(17)
    bits = finite_bits(rng, (2048, 4096))
    p = swap.to_device_radix(oracle_dict(bits, "sip"), cuda)
    twin = swap.to_device_twin(bf16_tensor(bits, cuda), device=cuda)
    assert tuple(twin["widths"]) == (3, 8)
    x = bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal(4096).astype(np.float32)), cuda)
    print("case twin plain linear", flush=True)
    assert torch.equal(radix_ops.gemv_fused(twin, x, None), radix_ops.gemv_fused(p, x, None))


@pytest.mark.parametrize("profile", ["sip", "gulp"])
def test_twin_matches_on_a_launch_long_enough_for_progress_balance(cuda, profile):
    """12288 x 4096 at M = 1 and 2: 192 blocks a workgroup, so the sip
    kernel's waves rebalance their priorities as they go (launches of 12 or
    more blocks a wave), in the twin as in the compressed kernel; the
    outputs stay bit for bit equal, and right."""
    import torch

    from drinkme_amd import radix_ops

    rng = np.random.default_rng(4096 + len(profile))
    R, C = 12288, 4096
    bits = finite_bits(rng, (R, C), spread=True)
    p, twin = _pair(bits, profile, cuda)
    xb = O.f32_to_bf16_bits(rng.standard_normal((2, C)).astype(np.float32))
    x = bf16_tensor(xb, cuda)
    print(f"case twin balanced launch {profile}", flush=True)
    y = radix_ops.gemv(p, x[0])
    assert torch.equal(radix_ops.gemv(twin, x[0]), y), "M=1"
    assert torch.equal(radix_ops.gemv_mc(twin, x), radix_ops.gemv_mc(p, x)), "M=2"
    ref, bound = O.gemv_f64(bits, O.bf16_bits_to_f32(xb[:1]))
    yy = y.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(yy - ref.reshape(yy.shape)) <= bound.reshape(yy.shape))
