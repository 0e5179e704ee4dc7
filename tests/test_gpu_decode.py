"""GPU parity: the dense decode (dmx_radix_decode) and the schedule
(dmx_radix_prepare) against the oracle, through the C ABI.

Mirrors drinkme's device gate bench/radix_gemv_bitpin.py:86-116 (all 65,536
bf16 patterns at every profile, 32- and 1024-weight blocks, bit-exact; the
schedule equal to the CPU one). The device reader over a short block against
the padded model (drinkme's tests/test_radix_bounds.py:149-182) is in
tests/test_gpu_bounds.py."""

import zlib

import numpy as np
import pytest

from oracle import radix_oracle as O
from tests.helpers import all_patterns, escape_heavy_bits, finite_bits, oracle_dict, u16_of

pytestmark = pytest.mark.gpu

PROFILES = ("sip", "balanced", "gulp")


@pytest.mark.parametrize("profile", PROFILES)
@pytest.mark.parametrize("block", [32, 1024])
def test_all_patterns_decode_exactly(cuda, profile, block):
    from drinkme_amd import radix_ops, swap

    bits = all_patterns()
    d = oracle_dict(bits, profile, block)
    rt = swap.to_device_radix(d, cuda)
    print(f"case all-patterns {profile} B{block}", flush=True)
    got = u16_of(radix_ops.decode_bits(rt))
    assert np.array_equal(got, bits)
    assert np.array_equal(u16_of(radix_ops.decode_bits(rt)), bits)  # deterministic
    if len(d["widths"]) > 2:
        want = O.schedule(O.Pack((512, 513), block, tuple(d["widths"]), d["rx_palette"], d["rx_offsets"],
                                 d["rx_data"]))
        assert np.array_equal(u16_of(rt["rx_schedule"]), want)


@pytest.mark.parametrize("shape", [(1, 1), (7, 33), (3, 1025), (129, 260), (17, 3079), (64, 4096), (8, 12288)])
@pytest.mark.parametrize("spread", [False, True])
def test_ragged_and_production_shapes_decode_exactly(cuda, shape, spread):
    from drinkme_amd import radix_ops, swap

    rng = np.random.default_rng(zlib.crc32(repr((shape, spread)).encode()))
    bits = finite_bits(rng, shape, spread)
    for profile in PROFILES:
        p = O.pack(bits, profile)
        if p.raw:
            continue
        d = oracle_dict(bits, profile)
        print(f"case ragged {shape} spread={spread} {profile}", flush=True)
        rt = swap.to_device_radix(d, cuda)
        assert np.array_equal(u16_of(radix_ops.decode_bits(rt)), bits)
        if len(d["widths"]) > 2:
            assert np.array_equal(u16_of(rt["rx_schedule"]), O.schedule(p))


@pytest.mark.parametrize("profile", ["sip", "gulp"])
def test_fast_decode_of_whole_block_tensors(cuda, profile):
    """Whole-block sip and gulp tensors decode on their GEMV kernel's work
    split (decode mode): every bf16 pattern laid out in whole blocks, and
    escape-heavy tensors (the terminal path, and for sip a terminal longer
    than 64 words; for gulp, tails longer than 64 words), each equal to the
    source and to the generic decoder."""
    from drinkme_amd import radix_ops, swap

    rng = np.random.default_rng(5 + len(profile))
    cases = {"all patterns": all_patterns((64, 2048)),
             "escapes 3%": escape_heavy_bits(rng, (300, 4096), 0.03),
             "escapes 45%": escape_heavy_bits(rng, (64, 4096), 0.45),
             "tall": finite_bits(rng, (2050, 2048), spread=True)}
    if profile == "gulp":
        # blocks whose tier-1, tier-2 and terminal words run past the one
        # word a lane loads (the exact path by the tail's length alone)
        from tests.test_gpu_gemv import _gulp_bits

        cases["long tail"] = _gulp_bits(rng, "long-tail", (300, 3072))
    for name, bits in cases.items():
        if O.pack(bits, profile).raw:
            continue
        print(f"case fast decode {profile} {name}", flush=True)
        rt = swap.to_device_radix(oracle_dict(bits, profile), cuda)
        fast = u16_of(radix_ops.decode_bits(rt))
        assert np.array_equal(fast, bits), f"{profile} {name}"
        prev = radix_ops.set_policy("generic")
        try:
            generic = u16_of(radix_ops.decode_bits(rt))
        finally:
            radix_ops.set_policy(prev)
        assert np.array_equal(generic, fast)
