"""CPU: the product's host side against the pinned oracle.

  - the threaded encoder in libdmx_radix.so (dmx_radix_native, the drop-in
    for drinkme's radix_native, src/drinkme/codec/radix_native.cpp:211-236)
    writes the golden bytes and the oracle's bytes, at every thread count;
  - its decoder and refusals (op 2; the reference's messages);
  - the raw fallback criterion (src/drinkme/codec/radix_pack.py:166-172);
  - the descriptor gate validate_radix (src/drinkme/codec/radix.py:174-238);
  - dmx_radix_pad_words = the widest block (the reach pad);
  - the synthetic weight streams: deterministic, thread-count independent,
    N(0, 0.02) and Student-t moments.
"""

import hashlib
import json
import os

import numpy as np
import pytest

from oracle import radix_oracle as O
from tests.helpers import all_patterns, finite_bits

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
PROFILES = ("sip", "balanced", "gulp")


@pytest.fixture(scope="module")
def rp():
    from drinkme_amd import radix_pack

    return radix_pack


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_product_encoder_writes_the_golden_bytes(rp):
    from tests.test_oracle_pinning import _golden_inputs

    with open(os.path.join(GOLDEN, "golden.json")) as f:
        cases = json.load(f)["cases"]
    inputs = _golden_inputs()
    for name, entry in cases.items():
        bits, _ = inputs[name]
        for profile, want in entry["profiles"].items():
            pal, off, data = rp.encode(bits, rp.widths_of(profile))
            assert pal.tolist() == want["palette"], (name, profile)
            assert _sha(off) == want["offsets_sha256"] and _sha(data) == want["data_sha256"], (name, profile)


@pytest.mark.parametrize("threads", [1, 3, 0])
@pytest.mark.parametrize("profile", PROFILES)
def test_product_encoder_equals_the_oracle_at_any_thread_count(rp, threads, profile):
    from drinkme_amd import _native

    rng = np.random.default_rng(41)
    bits = finite_bits(rng, (67, 5000), spread=True)
    prev = _native.lib().dmx_set_host_threads(threads)
    try:
        pal, off, data = rp.encode(bits, rp.widths_of(profile))
    finally:
        _native.lib().dmx_set_host_threads(prev)
    o = O.pack(bits, profile, allow_raw=False)
    assert np.array_equal(pal, o.palette) and np.array_equal(off, o.offsets) and np.array_equal(data, o.data)
    assert np.array_equal(rp.decode(pal, off, data, 67, 5000, rp.widths_of(profile)), bits)


@pytest.mark.parametrize("profile", PROFILES)
def test_product_codec_round_trips_all_bit_patterns(rp, profile):
    bits = all_patterns()
    d = rp.pack_array_radix(bits, profile)
    assert d is not None and d["bpw"] < 16
    assert np.array_equal(rp.decode(d["rx_palette"], d["rx_offsets"], d["rx_data"], 512, 513, d["widths"]), bits)
    rp.validate_radix(d)


def test_raw_fallback_matches_the_oracle_criterion(rp):
    rng = np.random.default_rng(19)
    noise = rng.integers(0, 65536, (128, 1024), dtype=np.uint16)
    assert rp.pack_array_radix(noise, "sip") is None
    assert O.pack(noise).raw
    d = rp.pack_weight_radix(noise, "sip")
    assert d["codec"] == "raw" and np.array_equal(d["raw_bits"], noise)
    tight = finite_bits(rng, (16, 1024))
    assert rp.pack_array_radix(tight, "sip") is not None and not O.pack(tight).raw


def test_product_decoder_refuses_a_cut_terminal_and_bad_palette(rp):
    bits = np.full((4, 1024), 0x3F80, np.uint16)
    bits[1, 100:140] = np.arange(40, dtype=np.uint16) << 7
    pal, off, data = rp.encode(bits, (3, 8))
    off2 = off.copy()
    off2[2:] -= 9
    cut = np.delete(data, np.s_[off2[2]:off2[2] + 9])
    with pytest.raises(ValueError):
        rp.decode(pal, off2, cut, 4, 1024, (3, 8))
    # decode trusts the palette, as drinkme's does (radix_native.cpp:173);
    # op 3 is the palette check, with the reference's wording
    codec = rp.HostCodec(4, 1024, (3, 8))
    codec.op(codec.CHECK_PALETTE, tables=rp.device_tables(pal, (3, 8)))
    for bad, why in ((np.zeros_like(pal), "invalid or repeated palette value"),):
        with pytest.raises(ValueError, match=why):
            codec.op(codec.CHECK_PALETTE, tables=rp.device_tables(bad, (3, 8)))
        if O.ref_available():
            with pytest.raises(ValueError, match=why):
                O._ref_call(3, None, 4, 1024, (3, 8), rp.device_tables(bad, (3, 8)), None)
    padded = rp.device_tables(pal, (3, 8))
    padded[7] = 9
    with pytest.raises(ValueError, match="nonzero palette padding"):
        codec.op(codec.CHECK_PALETTE, tables=padded)


def _dict(rp, bits, profile="gulp"):
    d = rp.pack_array_radix(bits, profile)
    assert d is not None
    return d


@pytest.mark.parametrize("field,value,why", [
    ("widths", [2, 4], "widths"), ("widths", [8, 8, 8], "alphabet"), ("block_size", 512 + 1, "block size"),
    ("R", 0, "shape"), ("rx_palette", np.zeros(21, np.uint8), "palette"),
    ("rx_offsets", np.zeros(5, np.uint32), "offsets"), ("rx_data", np.zeros(3, np.uint16), "payload")])
def test_validate_radix_refuses_by_name(rp, field, value, why):
    d = _dict(rp, np.full((4, 1024), 0x3F80, np.uint16))
    rp.validate_radix(d)
    with pytest.raises(ValueError, match=why):
        rp.validate_radix(dict(d, **{field: value}))


def test_validate_radix_refuses_blocks_outside_their_bounds(rp):
    d = _dict(rp, np.full((4, 1024), 0x3F80, np.uint16))
    off = d["rx_offsets"].copy()
    off[1] = 1
    with pytest.raises(ValueError, match=r"block 0 holds 1 word\(s\), fewer than the 320 its literal plane and "
                                         r"first tier take for 1024 weights"):
        rp.validate_radix(dict(d, rx_offsets=off))
    grown = d["rx_offsets"].astype(np.int64)
    grown[1:] += 500
    with pytest.raises(ValueError, match="holds 820 words, more than the 768 any block of 1024 weights can use"):
        rp.validate_radix(dict(d, rx_offsets=grown.astype(np.uint32),
                               rx_data=np.zeros(int(grown[-1]), np.uint32)))


@pytest.mark.parametrize("profile,pad", [("sip", 608), ("balanced", 672), ("gulp", 768)])
def test_pad_words_is_the_widest_block(rp, profile, pad):
    from drinkme_amd import _native

    w = np.array(rp.widths_of(profile), np.uint32)
    assert _native.lib().dmx_radix_pad_words(1024, w.ctypes.data, w.size) == pad
    assert rp.pad_words(rp.widths_of(profile)) == pad
    assert int(O.block_word_bounds(1024, rp.widths_of(profile))[1]) == pad
    for b in (32, 256, 4096):
        assert _native.lib().dmx_radix_pad_words(b, w.ctypes.data, w.size) == \
            int(O.block_word_bounds(b, rp.widths_of(profile))[1])


def test_padded_tables_index_a_zero_byte_on_the_escape_code(rp):
    pal = np.arange(1, 22, dtype=np.uint8)
    words = rp.padded_palette_words(pal, (2, 2, 4, 8))
    assert np.array_equal(words, O.padded_palette_words(pal, (2, 2, 4, 8)))
    b = words.view(np.uint8)
    assert b.size == 24 and b[3] == 0 and b[7] == 0 and b[8 + 15] == 0
    assert b[:3].tolist() == [1, 2, 3] and b[4:7].tolist() == [4, 5, 6] and b[8:23].tolist() == list(range(7, 22))


def test_synthetic_streams_are_deterministic_and_thread_independent():
    from drinkme_amd import _native, synth

    a = synth.weight("t", 0, "w", 300, 1000)
    prev = _native.lib().dmx_set_host_threads(1)
    try:
        b = synth.weight("t", 0, "w", 300, 1000)
    finally:
        _native.lib().dmx_set_host_threads(prev)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, synth.weight("t", 1, "w", 300, 1000))
    # a prefix of a longer draw of the same stream is the shorter draw
    assert np.array_equal(synth.bf16_bits(("t", 0, "w"), (300 * 1000 + 7,))[:300 * 1000], a.reshape(-1))


def test_synthetic_distributions():
    from drinkme_amd import synth

    w = O.bf16_bits_to_f32(synth.weight("t", 0, "n", 1024, 1024)).astype(np.float64)
    assert abs(w.mean()) < 1e-4 and abs(w.std() - 0.02) < 2e-4
    t = O.bf16_bits_to_f32(synth.weight("t", 0, "t4", 1024, 1024, synth.STUDENT_T4)).astype(np.float64)
    # t(4) * 0.02 / sqrt(2): std 0.02, heavy tails (kurtosis infinite; the
    # sample's is far above the normal's 3)
    assert abs(t.std() - 0.02) < 2e-3
    assert ((t - t.mean()) ** 4).mean() / t.var() ** 2 > 6
    x = O.bf16_bits_to_f32(synth.activation("t", "x", 4, 4096)).astype(np.float64)
    assert abs(x.std() - 1.0) < 0.05
    # bf16 round-to-nearest-even of a float32 value: every pattern is finite
    assert np.all(np.isfinite(w)) and np.all(np.isfinite(t))


def test_qwen3_8b_step_has_253_gemvs_and_7_57g_weights():
    from drinkme_amd import synth

    step = synth.qwen3_8b_step()
    assert len(step) == 253
    assert sum(r * c for _, _, r, c in step) == 36 * 192_937_984 + 151936 * 4096


def test_device_tables_layout_closed_form(rp):
    """Each nonterminal tier of width w takes ((1 << w) + 2) // 4 words
    (src/drinkme/codec/radix_pack.py:333-350), its 2^w - 1 entries first
    and zeros after, so the escape code 2^w - 1 reads a zero byte."""
    rng = np.random.default_rng(5)
    for widths in [(w, 8) for w in range(1, 9)] + [(2, 3, 8), (2, 2, 4, 8), (1, 4, 2, 8)]:
        assert rp.table_words(widths) == sum(((1 << w) + 2) // 4 for w in widths[:-1])
        cov = rp.covered_of(widths)
        pal = rng.permutation(256)[:cov].astype(np.uint8) if cov <= 256 else None
        if pal is None:
            continue
        t = rp.device_tables(pal, widths)
        assert t.size == 4 * rp.table_words(widths)
        at = base = 0
        for w in widths[:-1]:
            n = (1 << w) - 1
            assert np.array_equal(t[at:at + n], pal[base:base + n])
            assert not t[at + n:at + 4 * (((1 << w) + 2) // 4)].any()
            assert t[at + n] == 0  # the escape code's byte
            at += 4 * (((1 << w) + 2) // 4)
            base += n
        assert np.array_equal(rp.palette_of_tables(t, widths), pal)
