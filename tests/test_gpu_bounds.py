"""GPU parity over short blocks and a guarded allocation: the device reader
against the padded model, through the C ABI.

drinkme's device readers bounds-check no payload read; the reach pad after
the payload is the safety contract (src/drinkme/codec/radix_gpu.py:13-27,
swap.py:84-95). Its guard-buffer gate (tests/test_radix_bounds.py:624-680)
and padded model (:149-182) are restated here for this build's kernels:

  - a directory whose blocks are cut short (a block that ends at its fixed
    streams, so the terminal is never read; a gulp block cut one word into
    tier 1; a block cut one word inside its terminal, whose last escapes
    then read the next block's first word, or the pad; and, below the
    descriptor gate, a whole block cut to 3 words and a one-word tensor)
    decodes to oracle.padded_decode: every read past the payload sees the
    pad's zeros, and every read past a block's end the words that follow
    it, as drinkme's unmasked readers take them
    (radix_kernel_gpu.py:313-316);
  - the allocation is payload | pad | 4096 sentinel words (0xFFFFFFFF, an
    exponent of 255 and a literal of 255 wherever one is read): no decoded
    bit and no GEMV sum may come from the sentinel; the gulp schedule the
    device prepares over the same allocation equals the oracle's;
  - the negative control: the same buffers with a 16-word pad before the
    sentinel DO surface sentinel bits on the block cut to 3 words (its
    literal plane alone reaches 256 words), so the check discriminates.
    Every read of the control stays inside the allocation: no kernel
    reaches more than 768 words past a block's start, and 16 + 4096 words
    follow the payload.

Both the whole-block tensors the sip and gulp kernels take (M = 1, 4, 8:
the v_dot2 and matrix-core paths) and a ragged tensor (two full blocks and
a 52-weight tail per row, the generic kernel) are covered. The runtime
dicts here are built over the raw arrays, without the descriptor gate, so
that the below-gate directories reach the kernels.
"""

import numpy as np
import pytest

from oracle import radix_oracle as O
from tests.helpers import bf16_tensor, finite_bits, planted_mistakes_rejected, u16_of

pytestmark = pytest.mark.gpu

SENTINEL_WORDS = 4096
SHORT_PAD = 16


def _pack(bits, profile):
    p = O.pack(bits, profile, allow_raw=False)
    O.validate(p)
    return p


def _cut_block(p: O.Pack, block: int, keep: int) -> O.Pack:
    """p with block `block` holding only its first `keep` words: the words
    after them leave the payload, and every later block starts that much
    earlier."""
    off = p.offsets.astype(np.int64)
    start, end = int(off[block]), int(off[block + 1])
    assert 0 < keep < end - start
    data = np.concatenate([p.data[:start + keep], p.data[end:]])
    off[block + 1:] -= end - start - keep
    return O.Pack(p.shape, p.block_size, p.widths, p.palette, off.astype(np.uint32), data)


def _fixed_words(p: O.Pack, block: int) -> int:
    nb = -(-p.shape[1] // p.block_size)
    n = min(p.block_size, p.shape[1] - (block % nb) * p.block_size)
    return int(O.block_word_bounds(n, p.widths)[0])


def _tiered_bits(rng, shape) -> np.ndarray:
    """bf16 bits whose exponents fill the gulp tiers in order: 92% over six
    (tiers 0 and 1), 6.5% over fifteen (tier 2), 1.5% over ten (the
    terminal; sip's terminal holds these and most of the fifteen). A ragged
    tail block gets a dozen terminal exponents."""
    R, C = shape
    u = rng.random((R, C))
    main = rng.choice(np.arange(120, 126), size=(R, C), p=[.4, .25, .15, .1, .06, .04])
    mid = rng.integers(105, 120, (R, C))
    tail = rng.integers(126, 136, (R, C))
    e = np.where(u < 0.92, main, np.where(u < 0.985, mid, tail))
    if C % 1024:
        e[-1, -12:] = tail[-1, -12:]
    bits = (e.astype(np.uint16) << 7) | rng.integers(0, 128, (R, C), dtype=np.uint16)
    return bits | (rng.integers(0, 2, (R, C), dtype=np.uint16) << 15)


def _terminal_start(p: O.Pack, block: int) -> int:
    """The word of block `block` its terminal stream starts at."""
    t = _fixed_words(p, block)
    if len(p.widths) > 2:
        h = int(O.schedule(p)[block])
        t += (h & 0xFF) + (h >> 8)
    return t


def _zeros_after(p: O.Pack, block: int, words: int) -> O.Pack:
    """p with `words` zero words inserted after block `block`: its decode
    of that block is a reader's that stops at the block's end."""
    off = p.offsets.astype(np.int64)
    end = int(off[block + 1])
    data = np.concatenate([p.data[:end], np.zeros(words, np.uint32), p.data[end:]])
    off[block + 1:] += words
    off[block + 1] -= words  # (the block itself keeps its end)
    return O.Pack(p.shape, p.block_size, p.widths, p.palette, off.astype(np.uint32), data)


def _guarded(p: O.Pack, profile: str, cuda, zero_words: int, with_schedule: bool = True) -> dict:
    """A runtime dict over payload | zero_words zeros | SENTINEL_WORDS of
    0xFFFFFFFF, the gate not applied. The descriptor's pad is everything
    after the payload (the kernels' one bound is that it covers their
    reach)."""
    import torch

    from drinkme_amd import radix_ops, radix_pack

    R, C = p.shape
    B = p.block_size
    data = np.concatenate([p.data.astype(np.uint32), np.zeros(zero_words, np.uint32),
                           np.full(SENTINEL_WORDS, 0xFFFFFFFF, np.uint32)])
    d = torch.from_numpy(data.view(np.int32)).to(cuda).view(torch.uint32)
    off = torch.from_numpy(p.offsets.astype(np.uint32).view(np.int32)).to(cuda).view(torch.uint32)
    pal = torch.from_numpy(radix_pack.padded_palette_words(p.palette, p.widths).view(np.int32)).to(cuda)
    pal = pal.view(torch.uint32)
    nblk = R * -(-C // B)
    if len(p.widths) > 2 and with_schedule:
        sched = radix_ops.prepare_schedule(d, off, C, p.widths, B, nblk)
    else:
        sched = torch.empty(0, dtype=torch.uint16, device=cuda)
    return {"rx_data": d, "rx_offsets": off, "rx_palette": pal, "rx_schedule": sched, "NW": int(p.data.size),
            "rx_pad_words": zero_words + SENTINEL_WORDS, "R": R, "C": C, "widths": tuple(p.widths),
            "block_size": B, "NBK": nblk, "codec": "radix", "profile": profile, "layout": 0}


def _cases(profile, C):
    """(name, pack) per short-block case over a 2-row tensor of C columns."""
    rng = np.random.default_rng(4242 + C + len(profile))
    p = _pack(finite_bits(rng, (2, C), spread=True), profile)
    nb = -(-C // 1024)
    last = 2 * nb - 1
    cases = {"terminal-inner": _cut_block(p, 1, _fixed_words(p, 1)),
             "terminal-last": _cut_block(p, last, _fixed_words(p, last))}
    if profile == "gulp":
        cases["tier1-inner"] = _cut_block(p, 1, _fixed_words(p, 1) + 1)
    # blocks cut one word inside their terminal: the escapes that lost their
    # bytes read the following words (the next block's; the last block's
    # are the pad's zeros). The tensor keeps the fast kernels' common path
    # (gulp: under 128 tier-1 escapes a block) with terminals of several
    # words. The inner case must discriminate: its decode differs from a
    # reader's that stops at the block's end
    pt = _pack(_tiered_bits(rng, (2, C)), profile)
    for tag, b in (("inner", 1), ("last", last)):
        ln = int(pt.offsets[b + 1]) - int(pt.offsets[b])
        assert ln - 1 > _terminal_start(pt, b), f"block {b} has no terminal to cut"
        q = _cut_block(pt, b, ln - 1)
        if tag == "inner":
            bounded = O.padded_decode(_zeros_after(q, b, 64))
            assert not np.array_equal(O.padded_decode(q), bounded), "terminal-cut-inner does not discriminate"
        cases[f"terminal-cut-{tag}"] = q
    if profile == "gulp":
        # the same tensor's block cut one word into tier 1 (on the fast
        # kernel's common path, unlike tier1-inner's spread tensor)
        q = _cut_block(pt, 1, _fixed_words(pt, 1) + 1)
        assert not np.array_equal(O.padded_decode(q), O.padded_decode(_zeros_after(q, 1, 64))), \
            "tier1-cut-inner does not discriminate"
        cases["tier1-cut-inner"] = q
    for name, q in cases.items():
        O.validate(q)  # these pass the descriptor gate
    # below the gate: blocks cut inside their literal plane. Tight exponents
    # (the most common one 2^-6), so the weights the pad supplies (palette
    # entry 0) move a GEMV far past its bound wherever the sentinel would
    # stand in for them
    q = _pack(finite_bits(rng, (2, C)), profile)
    if C % 1024 == 0:
        cases["literal-last-full"] = _cut_block(q, 2 * nb - 1, 3)  # a whole block cut to 3 words
        cases["one-word"] = O.Pack((1, 1024), 1024, q.widths, q.palette, np.array([0, 1], np.uint32),
                                   np.zeros(1, np.uint32))
    else:
        cases["literal-last"] = _cut_block(q, last, 3)  # the ragged tail cut to 3 words
        cases["literal-full"] = _cut_block(q, last - 1, 3)  # the last row's second full block
    return cases


def _gemv_check(cuda, rt, expect, ms, what):
    import torch

    from drinkme_amd import radix_ops

    R, C = expect.shape
    rng = np.random.default_rng(R * 7 + C)
    for M in ms:
        xb = O.f32_to_bf16_bits(rng.standard_normal((M, C)).astype(np.float32))
        xf = O.bf16_bits_to_f32(xb)
        y = radix_ops.gemv_rows(rt, bf16_tensor(xb, cuda), None, torch.float32).cpu().numpy().astype(np.float64)
        ref, bound = O.gemv_f64(expect, xf)
        err = np.abs(y - ref) / bound
        assert np.all(err <= 1.0), f"{what} M={M}: the GEMV read past the pad (err/bound {err.max():.3g})"
        planted = planted_mistakes_rejected(y[0], expect, xf[0], 0)
        assert planted is None or min(planted) > 1.0, f"{what} M={M}: a planted mistake passed ({planted})"


@pytest.mark.parametrize("profile", ["sip", "gulp"])
@pytest.mark.parametrize("C", [2048, 2100])
def test_short_blocks_read_inside_the_pad(cuda, profile, C):
    from drinkme_amd import radix_ops

    for name, p in _cases(profile, C).items():
        print(f"case bounds {profile} C={C} {name}", flush=True)
        expect = O.padded_decode(p)
        pad = int(O.block_word_bounds(p.block_size, p.widths)[1])
        rt = _guarded(p, profile, cuda, pad)
        got = u16_of(radix_ops.decode_bits(rt))
        assert np.array_equal(got, expect), f"{profile} {name}: the decode read past the pad"
        if len(p.widths) > 2:
            assert np.array_equal(u16_of(rt["rx_schedule"]), O.schedule(p)), f"{profile} {name}: schedule"
        _gemv_check(cuda, rt, expect, (1, 4, 8), f"{profile} C={C} {name}")
        prev = radix_ops.set_policy("generic")
        try:
            assert np.array_equal(u16_of(radix_ops.decode_bits(rt)), expect), f"{profile} {name}: generic decode"
            _gemv_check(cuda, rt, expect, (1,), f"{profile} C={C} {name} generic")
        finally:
            radix_ops.set_policy(prev)


@pytest.mark.parametrize("profile", ["sip", "gulp"])
@pytest.mark.parametrize("C", [2048, 2100])
def test_a_short_pad_surfaces_the_sentinel(cuda, profile, C):
    """The negative control: with 16 zero words before the sentinel, the
    block cut to 3 words decodes sentinel bits (the fast kernel and the
    generic one), and the GEMV over it leaves the bound."""
    import torch

    from drinkme_amd import radix_ops

    # (a 52-weight tail cut to 3 words reaches 18 words: inside 16 + its own
    # 3, so the ragged control cuts a full block)
    name = "literal-last-full" if C % 1024 == 0 else "literal-full"
    p = _cases(profile, C)[name]
    expect = O.padded_decode(p)
    print(f"case bounds control {profile} C={C} {name}", flush=True)
    rt = _guarded(p, profile, cuda, SHORT_PAD)
    for policy in ("auto", "generic"):
        prev = radix_ops.set_policy(policy)
        try:
            got = u16_of(radix_ops.decode_bits(rt))
            assert not np.array_equal(got, expect), f"{profile} {policy}: a 16-word pad must not pass"
            xb = O.f32_to_bf16_bits(np.ones((1, p.shape[1]), np.float32))
            y = radix_ops.gemv_rows(rt, bf16_tensor(xb, cuda), None, torch.float32).cpu().numpy()
            ref, bound = O.gemv_f64(expect, O.bf16_bits_to_f32(xb))
            assert not np.all(np.abs(y - ref) <= bound), f"{profile} {policy}: the GEMV must leave the bound"
        finally:
            radix_ops.set_policy(prev)


def test_a_flipped_bit_fails_the_bit_check(cuda):
    """The bit gate's own negative control (drinkme's --selftest,
    bench/radix_gemv_bitpin.py:29-31): one decoded bit flipped after the
    kernel must fail the equality every decode test uses."""
    from drinkme_amd import radix_ops, swap
    from tests.helpers import oracle_dict

    rng = np.random.default_rng(31)
    bits = finite_bits(rng, (16, 2048), spread=True)
    rt = swap.to_device_radix(oracle_dict(bits, "sip"), cuda)
    got = u16_of(radix_ops.decode_bits(rt))
    assert np.array_equal(got, bits)
    for k in (0, 7, 15):  # a mantissa, an exponent and the sign bit
        bad = got.copy()
        bad[5, 1000] ^= np.uint16(1 << k)
        assert not np.array_equal(bad, bits)
