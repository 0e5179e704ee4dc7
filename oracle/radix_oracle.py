"""ORACLE — test infrastructure only (the checker, never the product).

A CPU restatement of drinkme's radix codec for bf16 weights: the C half
(oracle/radix_oracle.c, built by oracle/Makefile into
oracle/_build/libradix_oracle.so) does the per-block work; this module holds
the numpy half (descriptor validation and the closed-form bounds) and the
ctypes glue. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import it.

Restated functions and what they follow (paths in the drinkme source tree):
  PROFILES, widths_of      src/drinkme/codec/radix.py:14-18 (bf16 widths)
  check_widths             src/drinkme/codec/radix.py:139-146
  block_word_bounds        src/drinkme/codec/radix.py:149-171
  validate                 src/drinkme/codec/radix.py:174-238
  pack                     src/drinkme/codec/radix.py:77-136 (pack_array),
                           raw criterion radix.py:126-133 and
                           radix_pack.py:166-172 (_would_expand)
  decode                   src/drinkme/codec/radix.py:241-278
  padded_decode            tests/test_radix_bounds.py:149-182
  schedule                 src/drinkme/codec/radix_pack.py:376-411
  padded_palette_words     src/drinkme/codec/radix_pack.py:333-350
  gemv_f64                 bench/parity_common.py:231-251 (float64 dot and
                           the bound 2e-6 |W|.|x| + 1e-7)
  gemv_f32                 src/drinkme/codec/swap.py:344-352 (CPU route:
                           decode then fp32-accumulate matmul)

Pinning (tests/test_oracle_*.py): the compiled drinkme C++ codec
(oracle/_ref, built from the drinkme source where it lies) writes the same
bytes and decodes the same bits; the committed golden digests in
tests/golden/ were written by that compiled codec; the known answers of the
drinkme tests (352..608 / 320..768 block words, 9 terminal words for 33
escapes, the refusal messages); decode(encode(W)) == W over all 65,536 bf16
bit patterns; and a brute-force float64 dot on tiny shapes.
"""

from __future__ import annotations

import ctypes as ct
import os
from dataclasses import dataclass, replace

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libradix_oracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libradix_native_ref.so")

MANT, EXP = 7, 8
DEFAULT_BLOCK = 1024
PROFILES = {"sip": (3, 8), "balanced": (2, 3, 8), "gulp": (2, 2, 4, 8)}

_lib = None
_ref = None


def widths_of(profile: str) -> tuple:
    if profile not in PROFILES:
        raise ValueError(f"unknown profile: {profile!r}")
    return PROFILES[profile]


def lib():
    """The oracle's C half; raises when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        L = ct.CDLL(LIB_PATH)
        p, u64, u32, sz = ct.c_void_p, ct.c_uint64, ct.c_uint32, ct.c_size_t
        L.orc_palette.argtypes = [p, u64, u64, p, u32, p, p, sz]
        L.orc_plan.argtypes = [p, u64, u64, u32, p, u32, p, p, p, p, sz]
        L.orc_encode.argtypes = [p, u64, u64, u32, p, u32, p, p, p, u64, p, sz]
        L.orc_decode.argtypes = [p, u32, p, p, u64, u64, u64, u32, p, u32, u64, u64, p, p, sz]
        L.orc_padded_decode.argtypes = [p, u32, p, p, u64, u64, u64, u32, p, u32, p, p, sz]
        L.orc_schedule.argtypes = [p, p, u64, u64, u64, u32, p, u32, p, p, sz]
        L.orc_gemv_f64.argtypes = [p, u64, u64, p, u64, p, p]
        L.orc_gemv_f32.argtypes = [p, u64, u64, p, u64, p, p]
        for f in ("orc_palette", "orc_plan", "orc_encode", "orc_decode", "orc_padded_decode",
                  "orc_schedule"):
            getattr(L, f).restype = ct.c_int
        L.orc_gemv_f64.restype = None
        L.orc_gemv_f32.restype = None
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data


def _err():
    return ct.create_string_buffer(256)


def check_widths(widths) -> int:
    """The palette's entry count `covered`, or ValueError (radix.py:139-146)."""
    widths = tuple(widths)
    if (len(widths) < 2 or len(widths) > 8 or widths[-1] != EXP
            or any(type(w) is not int or w < 1 or w > 8 for w in widths)):
        raise ValueError("radix needs 2..8 widths in 1..8, ending with the exponent width")
    covered = sum((1 << w) - 1 for w in widths[:-1])
    if covered > 1 << EXP:
        raise ValueError("radix tiers exceed the exponent alphabet")
    return covered


def block_word_bounds(n, widths) -> tuple:
    """(fewest, most) u32 words a block of `n` weights can occupy: the fixed
    literal plane and first tier, then every data-dependent stream at its
    widest (radix.py:149-171)."""
    n = np.asarray(n, dtype=np.int64)
    fixed = (n * (MANT + 1) + 31) // 32 + (n * widths[0] + 31) // 32
    most = fixed + sum((n * w + 31) // 32 for w in widths[1:-1]) + (n * EXP + 31) // 32
    return fixed, most


def padded_table_bytes(widths) -> int:
    return sum(4 * (((1 << w) + 2) // 4) for w in widths[:-1])


@dataclass(frozen=True)
class Pack:
    """The codec's three arrays (radix.RadixPack's fields) for bf16."""
    shape: tuple
    block_size: int
    widths: tuple
    palette: np.ndarray
    offsets: np.ndarray
    data: np.ndarray
    raw: bool = False

    @property
    def nbytes(self) -> int:
        return self.palette.nbytes + self.offsets.nbytes + self.data.nbytes


def pack(bits: np.ndarray, profile: str = "sip", block_size: int = DEFAULT_BLOCK, widths=None,
         allow_raw: bool = True) -> Pack:
    """Encode u16 bf16 bit patterns; a tensor that would expand comes back
    raw (radix.py:77-136) unless allow_raw is False (the encoder's streams
    whatever their size, as radix_native.cpp's plan + encode write them).
    The round trip is checked before returning."""
    bits = np.asarray(bits)
    if bits.dtype != np.uint16 or bits.ndim != 2 or min(bits.shape) <= 0:
        raise ValueError("expected a nonempty 2D uint16 array of bf16 bit patterns")
    if type(block_size) is not int or block_size < 32 or block_size > 4096 or block_size & (block_size - 1):
        raise ValueError("block_size must be a power of two from 32 through 4096")
    widths = tuple(widths_of(profile) if widths is None else widths)
    covered = check_widths(widths)
    bits = np.ascontiguousarray(bits)
    R, C = bits.shape
    L = lib()
    w = np.array(widths, dtype=np.uint32)
    e = _err()
    palette = np.zeros(max(covered, 1), dtype=np.uint8)
    if L.orc_palette(_ptr(bits), R, C, _ptr(w), len(w), _ptr(palette), e, len(e)):
        raise ValueError(e.value.decode())
    palette = palette[:covered].copy()
    nb = (C + block_size - 1) // block_size
    offsets = np.zeros(R * nb + 1, dtype=np.uint32)
    words = ct.c_uint64()
    if L.orc_plan(_ptr(bits), R, C, block_size, _ptr(w), len(w), _ptr(palette), _ptr(offsets),
                  ct.byref(words), e, len(e)):
        raise ValueError(e.value.decode())
    data = np.zeros(words.value, dtype=np.uint32)
    if L.orc_encode(_ptr(bits), R, C, block_size, _ptr(w), len(w), _ptr(palette), _ptr(offsets),
                    _ptr(data), words.value, e, len(e)):
        raise ValueError(e.value.decode())
    p = Pack((R, C), block_size, widths, palette, offsets, data)
    device = data.nbytes + offsets.nbytes + padded_table_bytes(widths)
    if allow_raw and max(p.nbytes, device) >= bits.nbytes:
        p = Pack((R, C), block_size, widths, np.empty(0, np.uint8), np.empty(0, np.uint32),
                 bits.copy(), raw=True)
    if not np.array_equal(decode(p), bits):
        raise ValueError("radix round-trip verification failed")
    return p


def validate(p: Pack) -> None:
    """Descriptor checks before any payload word is read (radix.py:174-238):
    palette entries unique and inside the alphabet, the directory monotone
    from 0 to the payload end, every block inside [fewest, most] words."""
    if len(p.shape) != 2 or any(type(n) is not int or n <= 0 for n in p.shape) or type(p.raw) is not bool:
        raise ValueError("invalid radix shape or raw flag")
    b = p.block_size
    if type(b) is not int or b < 32 or b > 4096 or b & (b - 1):
        raise ValueError("invalid radix block size")
    covered = check_widths(p.widths)
    if p.palette.ndim != 1 or p.palette.dtype != np.uint8:
        raise ValueError("invalid radix palette")
    if p.offsets.ndim != 1 or p.offsets.dtype != np.uint32:
        raise ValueError("invalid radix directory")
    if p.raw:
        if p.data.shape != p.shape or p.data.dtype != np.uint16 or p.offsets.size or p.palette.size:
            raise ValueError("invalid raw radix tensor")
        return
    R, C = p.shape
    per_row = (C + b - 1) // b
    nb = R * per_row
    if p.palette.size != covered or len(np.unique(p.palette)) != covered:
        raise ValueError("invalid radix palette entries")
    if p.data.ndim != 1 or p.data.dtype != np.uint32:
        raise ValueError("invalid radix payload")
    off = p.offsets
    if off.size != nb + 1 or off[0] != 0 or off[-1] != p.data.size or np.any(off[1:] <= off[:-1]):
        raise ValueError("invalid radix block offsets")
    n = np.minimum(b, C - np.arange(nb, dtype=np.int64) % per_row * b)
    length = off[1:].astype(np.int64) - off[:-1].astype(np.int64)
    fewest, most = block_word_bounds(n, p.widths)
    short = np.flatnonzero(length < fewest)
    if short.size:
        i = int(short[0])
        raise ValueError(f"invalid radix block offsets: block {i} holds {int(length[i])} word(s), "
                         f"fewer than the {int(fewest[i])} its literal plane and first tier "
                         f"take for {int(n[i])} weights")
    long = np.flatnonzero(length > most)
    if long.size:
        i = int(long[0])
        raise ValueError(f"invalid radix block offsets: block {i} holds {int(length[i])} words, "
                         f"more than the {int(most[i])} any block of {int(n[i])} weights can use")


def decode(p: Pack) -> np.ndarray:
    """The CPU decoder: validate, then every block walked with its stream
    checks (radix.py:241-278)."""
    validate(p)
    if p.raw:
        return p.data.copy()
    R, C = p.shape
    out = np.empty((R, C), dtype=np.uint16)
    w = np.array(p.widths, dtype=np.uint32)
    data = np.ascontiguousarray(p.data, dtype=np.uint32)
    off = np.ascontiguousarray(p.offsets, dtype=np.uint32)
    pal = np.ascontiguousarray(p.palette, dtype=np.uint8)
    e = _err()
    if lib().orc_decode(_ptr(pal), pal.size, _ptr(off), _ptr(data), data.size, R, C, p.block_size,
                        _ptr(w), len(w), 0, R, _ptr(out), e, len(e)):
        raise ValueError(e.value.decode())
    return out


def decode_rows(p: Pack, first: int, rows: int, out: np.ndarray) -> None:
    """decode() over rows [first, first + rows) into `out` (rows x C), no
    validation — the bench's bounded CPU sample."""
    R, C = p.shape
    w = np.array(p.widths, dtype=np.uint32)
    e = _err()
    if lib().orc_decode(_ptr(p.palette), p.palette.size, _ptr(p.offsets), _ptr(p.data), p.data.size,
                        R, C, p.block_size, _ptr(w), len(w), first, rows, _ptr(out), e, len(e)):
        raise ValueError(e.value.decode())


def padded_decode(p: Pack) -> np.ndarray:
    """What the device reader produces over any gate-passing directory
    (tests/test_radix_bounds.py:149-182)."""
    R, C = p.shape
    out = np.empty((R, C), dtype=np.uint16)
    w = np.array(p.widths, dtype=np.uint32)
    data = np.ascontiguousarray(p.data, dtype=np.uint32)
    e = _err()
    if lib().orc_padded_decode(_ptr(p.palette), p.palette.size, _ptr(p.offsets), _ptr(data), data.size,
                               R, C, p.block_size, _ptr(w), len(w), _ptr(out), e, len(e)):
        raise ValueError(e.value.decode())
    return out


def schedule(p: Pack):
    """The per-block u16 stream-length header, or None for a two-tier
    profile (radix_pack.py:376-411)."""
    if len(p.widths) <= 2:
        return None
    R, C = p.shape
    nb = (C + p.block_size - 1) // p.block_size
    out = np.zeros(R * nb, dtype=np.uint16)
    w = np.array(p.widths, dtype=np.uint32)
    e = _err()
    if lib().orc_schedule(_ptr(p.offsets), _ptr(p.data), p.data.size, R, C, p.block_size, _ptr(w), len(w),
                          _ptr(out), e, len(e)):
        raise ValueError(e.value.decode())
    return out


def padded_palette_words(palette: np.ndarray, widths) -> np.ndarray:
    """Each nonterminal tier's (1 << w) - 1 entries zero-padded to whole u32
    words, tiers concatenated (radix_pack.py:333-350)."""
    parts, base = [], 0
    for w in widths[:-1]:
        n = (1 << w) - 1
        t = np.zeros(((n + 3) // 4) * 4, dtype=np.uint8)
        t[:n] = palette[base:base + n]
        parts.append(t.view(np.uint32))
        base += n
    return np.concatenate(parts)


def gemv_f64(bits: np.ndarray, x: np.ndarray):
    """(y, bound) float64 [M, R]: y = x . W^T, bound = 2e-6 |x|.|W|^T + 1e-7."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    R, C = bits.shape
    M = x.shape[0]
    y = np.empty((M, R), dtype=np.float64)
    bound = np.empty((M, R), dtype=np.float64)
    lib().orc_gemv_f64(_ptr(bits), R, C, _ptr(x), M, _ptr(y), _ptr(bound))
    return y, bound


def gemv_f32(bits: np.ndarray, x: np.ndarray, bias=None) -> np.ndarray:
    """fp32 [M, R]: the decoded weight times fp32 x with fp32 accumulation,
    the bias (fp32) added before the caller's one rounding."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    R, C = bits.shape
    M = x.shape[0]
    y = np.empty((M, R), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().orc_gemv_f32(_ptr(bits), R, C, _ptr(x), M, _ptr(b), _ptr(y))
    return y


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bits (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)


# ---------------------------------------------------------------------------
# The compiled drinkme codec (oracle/_ref): built from its own source file by
# `make -C oracle ref` where the drinkme tree exists, and used only to pin
# this restatement and as the CPU baseline's reference decoder.

def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref_lib():
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"reference codec not built: {REF_PATH}")
        L = ct.CDLL(REF_PATH)
        p, u64, u32 = ct.c_void_p, ct.c_uint64, ct.c_uint32
        L.radix_native.argtypes = [u32, p, u64, u64, u64, u64, u32, u32, p, u32, p, p, p, u64, u64, u64,
                                   p, p, u64]
        L.radix_native.restype = ct.c_int
        _ref = L
    return _ref


def _ref_call(op, value, R, C, widths, tables, offsets, data=None, first=0, rows=0):
    w = np.ascontiguousarray(np.asarray(widths, dtype=np.uint32))
    err = ct.create_string_buffer(1024)
    res = ct.c_uint64()
    nb = (C + 1023) // 1024
    status = ref_lib().radix_native(op, _ptr(value), R, C, R, nb, 7, 8, _ptr(w), len(w), _ptr(tables),
                                    _ptr(offsets), _ptr(data), 0 if data is None else data.size, first,
                                    rows, ct.byref(res), err, len(err))
    if status:
        raise ValueError("reference radix: " + err.value.decode())
    return res.value


def ref_encode(bits: np.ndarray, widths):
    """The compiled drinkme encoder (1024-weight blocks, one palette region):
    (palette u8 unpadded, offsets u32, data u32)."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    R, C = bits.shape
    nb = (C + 1023) // 1024
    tables = np.zeros(padded_table_bytes(widths), dtype=np.uint8)
    offsets = np.zeros(R * nb + 1, dtype=np.uint32)
    words = _ref_call(0, bits, R, C, widths, tables, offsets)
    data = np.zeros(words, dtype=np.uint32)
    _ref_call(1, bits, R, C, widths, tables, offsets, data)
    parts, at = [], 0
    for w in widths[:-1]:
        n = (1 << w) - 1
        parts.append(tables[at:at + n])
        at += ((n + 3) // 4) * 4
    return np.concatenate(parts).astype(np.uint8), offsets, data


def ref_decode(palette, offsets, data, R, C, widths, first=0, rows=None, out=None) -> np.ndarray:
    """The compiled drinkme decoder over rows [first, first + rows)."""
    rows = R - first if rows is None else rows
    tables = np.zeros(padded_table_bytes(widths), dtype=np.uint8)
    at = base = 0
    for w in widths[:-1]:
        n = (1 << w) - 1
        tables[at:at + n] = palette[base:base + n]
        at += ((n + 3) // 4) * 4
        base += n
    if out is None:
        out = np.empty((rows, C), dtype=np.uint16)
    _ref_call(2, out, R, C, widths, tables, np.ascontiguousarray(offsets, dtype=np.uint32),
              np.ascontiguousarray(data, dtype=np.uint32), first, rows)
    return out


__all__ = ["PROFILES", "Pack", "pack", "decode", "decode_rows", "padded_decode", "validate", "schedule",
           "block_word_bounds", "check_widths", "widths_of", "padded_palette_words", "gemv_f64", "gemv_f32",
           "bf16_bits_to_f32", "f32_to_bf16_bits", "ref_available", "ref_encode", "ref_decode", "replace"]
