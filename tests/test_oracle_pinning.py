"""CPU: pins the oracle before anything is checked against it.

  - the golden digests in tests/golden/, written by drinkme's own C++ codec
    (src/drinkme/codec/radix_native.cpp, compiled from its source file):
    the oracle's encoder writes the same palette, directory and payload;
  - the compiled drinkme codec itself (oracle/_ref), where it is built:
    same bytes on fresh seeded inputs, and each decodes the other's;
  - drinkme's known answers (tests/test_radix.py, docs/pack-format.md:
    296-302): block bounds 352..608 (sip) and 320..768 (gulp) words, 9
    terminal words for the 40-exponent block, the refusal wording;
  - closed forms and brute force: decode(encode(W)) == W over all 65,536
    bf16 patterns, the float64 dot against math.fsum, the padded reader's
    answer on a cut terminal (the escaped exponents read as zero).
"""

import hashlib
import json
import math
import os

import numpy as np
import pytest

from oracle import radix_oracle as O
from tests.helpers import all_patterns, finite_bits

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
PROFILES = ("sip", "balanced", "gulp")


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _golden():
    with open(os.path.join(GOLDEN, "golden.json")) as f:
        return json.load(f)["cases"]


def _golden_inputs():
    """The inputs tests/golden/make_golden.py encoded, rebuilt from the same
    seeds; the source digest in the fixture proves they are the same bits."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLDEN, "make_golden.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return {name: (bits, profiles) for name, bits, profiles in mod.cases()}


@pytest.fixture(scope="module")
def golden_inputs():
    return _golden_inputs()


@pytest.mark.parametrize("case", sorted(_golden()))
def test_oracle_encoder_writes_the_golden_bytes(golden_inputs, case):
    entry = _golden()[case]
    bits, _ = golden_inputs[case]
    assert list(bits.shape) == entry["shape"] and _sha(bits) == entry["source_sha256"]
    for profile, want in entry["profiles"].items():
        p = O.pack(bits, profile, allow_raw=False)
        assert p.palette.tolist() == want["palette"], (case, profile)
        assert p.data.size == want["words"], (case, profile)
        assert _sha(p.offsets) == want["offsets_sha256"], (case, profile)
        assert _sha(p.data) == want["data_sha256"], (case, profile)
        assert _sha(p.palette) == want["palette_sha256"]


@pytest.mark.parametrize("profile", PROFILES)
def test_oracle_decodes_the_golden_arrays(profile):
    z = np.load(os.path.join(GOLDEN, "small.npz"))
    bits = z["bits"]
    p = O.Pack(bits.shape, 1024, O.PROFILES[profile], z[f"{profile}_palette"], z[f"{profile}_offsets"],
               z[f"{profile}_data"])
    assert np.array_equal(O.decode(p), bits)
    assert np.array_equal(O.padded_decode(p), bits)
    mine = O.pack(bits, profile, allow_raw=False)
    for got, want in ((mine.palette, p.palette), (mine.offsets, p.offsets), (mine.data, p.data)):
        assert np.array_equal(got, want)


needs_ref = pytest.mark.skipif(not O.ref_available(), reason="compiled drinkme codec not built (make -C oracle ref)")


@needs_ref
@pytest.mark.parametrize("shape", [(1, 1), (5, 31), (7, 1025), (64, 4096), (3, 12288)])
@pytest.mark.parametrize("spread", [False, True])
@pytest.mark.parametrize("profile", PROFILES)
def test_oracle_equals_the_compiled_reference(shape, spread, profile):
    rng = np.random.default_rng(sum(shape) * 7 + spread)
    bits = finite_bits(rng, shape, spread)
    pal, off, data = O.ref_encode(bits, O.PROFILES[profile])
    mine = O.pack(bits, profile, allow_raw=False)
    assert np.array_equal(mine.palette, pal)
    assert np.array_equal(mine.offsets, off)
    assert np.array_equal(mine.data, data)
    assert np.array_equal(O.ref_decode(mine.palette, mine.offsets, mine.data, *shape, O.PROFILES[profile]), bits)
    ref_pack = O.Pack(shape, 1024, O.PROFILES[profile], pal, off, data)
    assert np.array_equal(O.decode(ref_pack), bits)
    if shape[0] > 2:  # a row range
        assert np.array_equal(O.ref_decode(pal, off, data, *shape, O.PROFILES[profile], first=1, rows=2),
                              bits[1:3])
        out = np.empty((2, shape[1]), np.uint16)
        O.decode_rows(ref_pack, 1, 2, out)
        assert np.array_equal(out, bits[1:3])


@needs_ref
@pytest.mark.parametrize("profile", PROFILES)
def test_schedule_is_the_reference_stream_lengths(profile):
    """The gulp/balanced schedule: byte (level - 1) = word length of tier
    `level`'s stream, read back from the compiled encoder's own blocks by
    walking their tier-0 codes (radix_pack.py:353-411)."""
    rng = np.random.default_rng(3)
    bits = finite_bits(rng, (9, 3000), spread=True)
    widths = O.PROFILES[profile]
    pal, off, data = O.ref_encode(bits, widths)
    p = O.Pack(bits.shape, 1024, widths, pal, off, data)
    sched = O.schedule(p)
    if len(widths) <= 2:
        assert sched is None
        return
    # closed form from the source: escapes per tier from the palette ranks
    rank = np.full(256, 255, np.int64)
    rank[pal] = np.arange(pal.size)
    exps = (bits >> 7) & 0xFF
    nb = (bits.shape[1] + 1023) // 1024
    want = []
    for r in range(bits.shape[0]):
        for b in range(nb):
            e = rank[exps[r, b * 1024:(b + 1) * 1024]]
            lens, base = [], 0
            for w in widths[:-1]:
                base += (1 << w) - 1
                lens.append(int(np.sum(e >= base)))
            # tier k (k >= 1) holds the codes of weights that escaped tiers < k
            words = [(lens[k - 1] * widths[k] + 31) // 32 for k in range(1, len(widths) - 1)]
            want.append(sum(wd << (8 * i) for i, wd in enumerate(words)))
    assert np.array_equal(sched.astype(np.int64), np.array(want))


@pytest.mark.parametrize("profile,fewest,most", [("sip", 352, 608), ("balanced", 320, 672), ("gulp", 320, 768)])
def test_block_word_bounds_known_answers(profile, fewest, most):
    assert tuple(int(v) for v in O.block_word_bounds(1024, O.PROFILES[profile])) == (fewest, most)


def test_forty_rare_exponents_take_nine_terminal_words():
    """tests/test_radix.py:56-68: 40 exponents past sip's 7-entry palette in
    one block take 9 terminal words; cutting them passes the directory gate
    and the decoder refuses the block. (The palette is 127 and the six
    smallest of the 40, so 34 escape: 272 bits, 9 words. drinkme's comment
    there counts 33, which gives the same 9 words.)"""
    bits = np.full((4, 1024), 0x3F80, np.uint16)
    bits[1, 100:140] = np.arange(40, dtype=np.uint16) << 7
    p = O.pack(bits, "sip")
    fewest, _ = O.block_word_bounds(1024, p.widths)
    terminal = int(p.offsets[2] - p.offsets[1] - fewest)
    assert terminal == 9
    off = p.offsets.copy()
    off[2:] -= terminal
    cut = O.replace(p, offsets=off, data=np.delete(p.data, np.s_[off[2]:off[2] + terminal]))
    O.validate(cut)
    with pytest.raises(ValueError, match="truncated radix stream"):
        O.decode(cut)
    if O.ref_available():
        with pytest.raises(ValueError):
            O.ref_decode(cut.palette, cut.offsets, cut.data, 4, 1024, p.widths)
    # the device reader over the cut block: the terminal is not read (its
    # end is where the stream would start), so the 34 escaped weights keep
    # sign and mantissa and read exponent 0; every other block is intact
    want = bits.copy()
    escaped = np.isin((bits[1] >> 7) & 0xFF, p.palette, invert=True)
    want[1, escaped] &= 0x807F
    assert escaped.sum() == 34
    assert np.array_equal(O.padded_decode(cut), want)


def test_a_block_cut_inside_its_literal_plane_is_refused_by_name():
    p = O.pack(np.full((4, 1024), 0x3F80, np.uint16), "gulp")
    off = p.offsets.copy()
    off[1] = 1
    with pytest.raises(ValueError, match="fewer than the 320 its literal plane"):
        O.decode(O.replace(p, offsets=off))
    with pytest.raises(ValueError, match="offsets"):
        O.decode(O.replace(p, offsets=p.offsets[:-1]))
    with pytest.raises(ValueError, match="palette"):
        O.decode(O.replace(p, palette=np.zeros_like(p.palette)))
    grown = p.offsets.copy()
    grown[1:] += 500
    with pytest.raises(ValueError, match="more than the 768"):
        O.validate(O.replace(p, offsets=grown, data=np.zeros(int(grown[-1]), np.uint32)))


@pytest.mark.parametrize("profile", PROFILES)
@pytest.mark.parametrize("block", [32, 1024])
def test_all_bit_patterns_round_trip_compressed(profile, block):
    bits = all_patterns()
    p = O.pack(bits, profile, block)
    assert not p.raw and p.nbytes < bits.nbytes
    assert np.array_equal(O.decode(p), bits)
    assert np.array_equal(O.padded_decode(p), bits)


@pytest.mark.parametrize("shape", [(1, 1), (1, 31), (7, 33), (3, 1023), (3, 1025), (2, 4101)])
@pytest.mark.parametrize("block", [32, 256, 1024, 4096])
def test_partial_rows_and_no_escape_streams(shape, block):
    src = np.full((shape[0], shape[1] * 2), 0x3F81, np.uint16)[:, ::2]
    p = O.pack(src, "gulp", block)
    assert np.array_equal(O.decode(p), src)
    assert p.nbytes <= src.nbytes


def test_random_bits_fall_back_raw_without_expansion():
    a = np.random.default_rng(19).integers(0, 65536, (128, 1024), dtype=np.uint16)
    p = O.pack(a)
    assert p.raw and p.nbytes == a.nbytes and np.array_equal(O.decode(p), a)


def test_deterministic_palette_and_bytes():
    a = np.tile(np.arange(65536, dtype=np.uint16), 4).reshape(256, 1024)
    a[:192] = 0x3F80
    one, two = O.pack(a), O.pack(a)
    for field in ("palette", "offsets", "data"):
        assert np.array_equal(getattr(one, field), getattr(two, field))


def test_palette_order_is_count_descending_ties_exponent_ascending():
    """radix_native.cpp:74-76: the palette is the exponents by count, most
    frequent first, equal counts in ascending exponent order."""
    counts = {130: 50, 120: 300, 121: 300, 119: 7, 118: 7, 117: 7, 116: 1, 125: 90, 140: 2}
    vals = np.concatenate([np.full(n, e << 7, np.uint16) for e, n in counts.items()])
    bits = np.random.default_rng(0).permutation(vals)[None, :]
    want = sorted(counts, key=lambda e: (-counts[e], e))[:7]
    assert O.pack(bits, "sip", allow_raw=False).palette.tolist() == want


@pytest.mark.parametrize("kwargs", [dict(block_size=31), dict(block_size=512.0), dict(widths=()),
                                    dict(widths=(2,)), dict(widths=(8, 8, 8)), dict(widths=(2, 0, 8)),
                                    dict(widths=(2, 4)), dict(profile="unknown")])
def test_invalid_parameters(kwargs):
    with pytest.raises(ValueError):
        O.pack(np.zeros((4, 1024), np.uint16), **kwargs)


@pytest.mark.parametrize("a", [np.zeros((0, 32), np.uint16), np.zeros(32, np.uint16),
                               np.zeros((32, 32), np.float32), np.zeros((32, 32), np.int16)])
def test_invalid_inputs(a):
    with pytest.raises(ValueError):
        O.pack(a)


def test_gemv_f64_is_the_exact_dot_with_its_bound():
    rng = np.random.default_rng(5)
    bits = finite_bits(rng, (5, 37), spread=True)
    x = rng.standard_normal((3, 37)).astype(np.float32)
    y, bound = O.gemv_f64(bits, x)
    w = O.bf16_bits_to_f32(bits).astype(np.float64)
    for m in range(3):
        for r in range(5):
            exact = math.fsum(float(a) * float(b) for a, b in zip(w[r], x[m].astype(np.float64)))
            assert abs(y[m, r] - exact) <= 1e-12 * math.fsum(abs(float(a) * float(b)) for a, b in zip(w[r], x[m]))
            assert bound[m, r] == pytest.approx(2e-6 * math.fsum(abs(float(a) * float(b))
                                                                 for a, b in zip(w[r], x[m])) + 1e-7, rel=1e-12)


def test_gemv_f32_accumulates_in_float32_in_column_order():
    """A sum whose float32 value depends on order: 1 + 2^-24 * 4 in column
    order is 1 (each small term rounds away); the oracle must give 1."""
    w = np.ones((1, 5), np.float32)
    bits = O.f32_to_bf16_bits(w)
    x = np.array([[1.0, 2.0 ** -24, 2.0 ** -24, 2.0 ** -24, 2.0 ** -24]], np.float32)
    assert O.gemv_f32(bits, x)[0, 0] == np.float32(1.0)
    assert O.gemv_f64(bits, x)[0][0, 0] == 1.0 + 4 * 2.0 ** -24
    b = O.gemv_f32(bits, x, np.array([-1.0], np.float32))
    assert b[0, 0] == np.float32(0.0)


def test_bf16_rounding_is_round_to_nearest_even():
    f = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20, -0.0, np.inf, np.nan],
                 np.float32)
    got = O.f32_to_bf16_bits(f)
    assert got[:6].tolist() == [0x3F80, 0x3F80, 0x3F82, 0x3F81, 0x8000, 0x7F80]
    assert (got[6] & 0x7F80) == 0x7F80 and (got[6] & 0x7F)
    assert np.array_equal(O.bf16_bits_to_f32(got[:6]), np.array([1.0, 1.0, 1.0 + 2 ** -6, 1.0 + 2 ** -7, -0.0,
                                                                np.inf], np.float32))
