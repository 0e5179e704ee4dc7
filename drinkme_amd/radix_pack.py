"""The radix codec as a pack tensor: profiles, the native encoder, the raw
fallback and the descriptor gate — the producer side of the kernels'
inputs, with drinkme's function names and dict layout
(src/drinkme/codec/radix_pack.py, src/drinkme/codec/radix.py:149-238).

A radix tensor dict (src/drinkme/codec/radix_pack.py:9-22):
    rx_palette  u8  [covered]      exponents in code order, unpadded
    rx_offsets  u32 [R * NB + 1]   word directory
    rx_data     u32 [NW]           concatenated block streams
    R, C, bpw, codec = "radix", profile, widths, block_size = 1024

Encoding runs on host threads in libdmx_radix.so (dmx_radix_native, the
drop-in for drinkme's radix_native) and is verified by decoding back before
the dict is returned, as drinkme's native encoder does
(src/drinkme/codec/radix_native.py:195-217).
"""

from __future__ import annotations

import ctypes as ct

import numpy as np

from . import _native

RADIX = "radix"
RAW = "raw"
PROFILES = ("sip", "balanced", "gulp")
PROFILE_WIDTHS = {"sip": (3, 8), "balanced": (2, 3, 8), "gulp": (2, 2, 4, 8)}
DEFAULT_PROFILE = "sip"
RADIX_BLOCK = 1024
MANT, EXP = 7, 8
ARRAYS_RADIX = ("rx_palette", "rx_offsets", "rx_data")


def widths_of(profile: str) -> tuple:
    if profile not in PROFILE_WIDTHS:
        raise ValueError(f"unknown profile {profile!r}; one of {PROFILES}")
    return PROFILE_WIDTHS[profile]


def is_radix_pack(p: dict) -> bool:
    return p.get("codec") == RADIX


def is_raw_pack(p: dict) -> bool:
    return p.get("codec") == RAW


def covered_of(widths) -> int:
    """Palette entries the nonterminal tiers address."""
    return sum((1 << int(w)) - 1 for w in tuple(widths)[:-1])


def table_words(widths) -> int:
    """u32 words of the padded device tables: ((1 << w) + 2) // 4 per tier."""
    return sum(((1 << int(w)) + 2) // 4 for w in tuple(widths)[:-1])


def block_word_bounds(n, widths):
    """(fewest, most) words a block of n weights occupies: the literal plane
    and tier 0 are fixed; later tiers and the terminal hold 0..n entries
    each (src/drinkme/codec/radix.py:149-171). `most` is also the reach
    pad the device allocation carries."""
    n = np.asarray(n, dtype=np.int64)
    w = [int(x) for x in widths]
    per = lambda k, width: (k * width + 31) // 32  # noqa: E731
    fewest = per(n, MANT + 1) + per(n, w[0])
    return fewest, fewest + sum(per(n, x) for x in w[1:])


def pad_words(widths, block: int = RADIX_BLOCK) -> int:
    return int(block_word_bounds(block, widths)[1])


def _native_call(op, value, R, C, widths, tables, offsets, data=None, first=0, rows=0):
    L = _native.lib()
    w = np.ascontiguousarray(np.asarray(widths, dtype=np.uint32))
    err = _native.error_buffer()
    res = ct.c_uint64()
    nb = (C + RADIX_BLOCK - 1) // RADIX_BLOCK
    ptr = lambda a: None if a is None else a.ctypes.data  # noqa: E731
    status = L.dmx_radix_native(op, ptr(value), R, C, R, nb, MANT, EXP, ptr(w), len(w), ptr(tables), ptr(offsets),
                                ptr(data), 0 if data is None else data.size, first, rows, ct.byref(res), err,
                                len(err))
    if status:
        raise ValueError("native radix: " + err.value.decode())
    return res.value


def _tables_from_palette(palette: np.ndarray, widths) -> np.ndarray:
    tables = np.zeros(4 * table_words(widths), dtype=np.uint8)
    at = base = 0
    for w in tuple(widths)[:-1]:
        n = (1 << int(w)) - 1
        tables[at:at + n] = palette[base:base + n]
        at += ((n + 3) // 4) * 4
        base += n
    return tables


def _palette_from_tables(tables: np.ndarray, widths) -> np.ndarray:
    parts, at = [], 0
    for w in tuple(widths)[:-1]:
        n = (1 << int(w)) - 1
        parts.append(tables[at:at + n])
        at += ((n + 3) // 4) * 4
    return np.concatenate(parts).astype(np.uint8)


def encode(U: np.ndarray, widths):
    """u16 [R, C] bf16 bits -> (palette u8 unpadded, offsets u32, data u32),
    1024-weight blocks, one palette per tensor; verified by decoding back."""
    U = np.ascontiguousarray(U, dtype=np.uint16)
    R, C = U.shape
    nb = (C + RADIX_BLOCK - 1) // RADIX_BLOCK
    tables = np.zeros(4 * table_words(widths), dtype=np.uint8)
    offsets = np.zeros(R * nb + 1, dtype=np.uint32)
    words = _native_call(0, U, R, C, widths, tables, offsets)
    data = np.zeros(words, dtype=np.uint32)
    _native_call(1, U, R, C, widths, tables, offsets, data)
    back = np.empty_like(U)
    _native_call(2, back, R, C, widths, tables, offsets, data, 0, R)
    if not np.array_equal(back, U):
        raise ValueError("native radix: CPU round trip differs from the source bits")
    return _palette_from_tables(tables, widths), offsets, data


def decode(palette, offsets, data, R: int, C: int, widths) -> np.ndarray:
    """The host decoder (dmx_radix_native op 2): u16 [R, C]."""
    nb = (C + RADIX_BLOCK - 1) // RADIX_BLOCK
    if offsets.ndim != 1 or offsets.size != R * nb + 1:
        raise ValueError("native radix: invalid radix block offsets")
    if palette.ndim != 1 or palette.size != covered_of(widths):
        raise ValueError("native radix: invalid radix palette entries")
    out = np.empty((R, C), dtype=np.uint16)
    _native_call(2, out, R, C, widths, _tables_from_palette(palette, widths),
                 np.ascontiguousarray(offsets, dtype=np.uint32), np.ascontiguousarray(data, dtype=np.uint32), 0, R)
    return out


def _would_expand(palette, offsets, data, widths, nbytes: int) -> bool:
    """The raw criterion: the stored bytes or the device bytes (tables padded
    to whole words) reach the raw plane's size
    (src/drinkme/codec/radix_pack.py:166-172)."""
    stored = palette.nbytes + offsets.nbytes + data.nbytes
    device = data.nbytes + offsets.nbytes + 4 * table_words(widths)
    return max(stored, device) >= nbytes


def pack_array_radix(U: np.ndarray, compression_profile: str) -> dict | None:
    """u16 [R, C] bf16 bits -> the radix tensor dict, or None when radix
    would not compress it (the caller stores it raw)
    (src/drinkme/codec/radix_pack.py:175-205)."""
    U = np.ascontiguousarray(U, dtype=np.uint16)
    if U.ndim != 2 or min(U.shape) < 1:
        raise ValueError("pack_array_radix: need a nonempty 2D uint16 array")
    widths = widths_of(compression_profile)
    palette, offsets, data = encode(U, widths)
    if _would_expand(palette, offsets, data, widths, U.nbytes):
        return None
    R, C = U.shape
    stored = palette.nbytes + offsets.nbytes + data.nbytes
    return {"rx_palette": palette, "rx_offsets": offsets, "rx_data": data, "R": int(R), "C": int(C),
            "bpw": 8.0 * stored / (R * C), "codec": RADIX, "profile": compression_profile,
            "widths": list(widths), "block_size": RADIX_BLOCK}


def raw_dict(U: np.ndarray) -> dict:
    """The raw fallback tensor: the bf16 bit patterns verbatim."""
    U = np.ascontiguousarray(U, dtype=np.uint16)
    if U.ndim != 2 or min(U.shape) < 1:
        raise ValueError("raw_dict: need a nonempty 2D uint16 array")
    R, C = U.shape
    return {"raw_bits": U, "R": int(R), "C": int(C), "bpw": 16.0, "codec": RAW}


def pack_weight_radix(U: np.ndarray, compression_profile: str) -> dict:
    """One tensor: the radix dict, or the raw dict when radix would expand
    it (src/drinkme/codec/radix_pack.py:217-236, over u16 bits)."""
    p = pack_array_radix(U, compression_profile)
    return raw_dict(U) if p is None else p


def padded_palette_words(palette: np.ndarray, widths) -> np.ndarray:
    """The device lookup tables: each nonterminal tier's entries in a
    zero-filled run of ceil(n / 4) words, tiers concatenated — the escape
    code indexes a zero byte (src/drinkme/codec/radix_pack.py:333-350)."""
    return _tables_from_palette(np.asarray(palette, dtype=np.uint8), widths).view(np.uint32)


def validate_radix(p: dict) -> None:
    """The descriptor gate before any device allocation: widths, block size,
    palette (unique entries), and the directory — strictly increasing from
    0 to the payload end, every block between its fixed streams and the
    widest block — with radix.validate's checks in its order and words
    (src/drinkme/codec/radix.py:174-238). Raises ValueError."""
    widths = tuple(int(w) for w in p["widths"])
    if (len(widths) < 2 or len(widths) > 8 or widths[-1] != EXP or any(w < 1 or w > 8 for w in widths)):
        raise ValueError("radix needs 2..8 widths in 1..8, ending with the exponent width")
    covered = covered_of(widths)
    if covered > 1 << EXP:
        raise ValueError("radix tiers exceed the exponent alphabet")
    B = int(p["block_size"])
    if B < 32 or B > 4096 or B & (B - 1):
        raise ValueError("invalid radix block size")
    R, C = int(p["R"]), int(p["C"])
    if R <= 0 or C <= 0:
        raise ValueError("invalid radix shape")
    palette = np.asarray(p["rx_palette"])
    if palette.ndim != 1 or palette.dtype != np.uint8:
        raise ValueError("invalid radix palette")
    offsets = np.asarray(p["rx_offsets"])
    if offsets.ndim != 1 or offsets.dtype != np.uint32:
        raise ValueError("invalid radix directory")
    if palette.size != covered or np.unique(palette).size != covered:
        raise ValueError("invalid radix palette entries")
    data = np.asarray(p["rx_data"])
    if data.ndim != 1 or data.dtype != np.uint32:
        raise ValueError("invalid radix payload")
    per_row = -(-C // B)
    if (offsets.size != R * per_row + 1 or offsets[0] != 0 or int(offsets[-1]) != data.size
            or np.any(offsets[1:] <= offsets[:-1])):
        raise ValueError("invalid radix block offsets")
    extent = np.diff(offsets.astype(np.int64))
    n = np.minimum(B, C - (np.arange(R * per_row, dtype=np.int64) % per_row) * B)
    fewest, most = block_word_bounds(n, widths)
    short = np.flatnonzero(extent < fewest)
    if short.size:
        i = int(short[0])
        raise ValueError(f"invalid radix block offsets: block {i} holds {int(extent[i])} word(s), fewer than the "
                         f"{int(fewest[i])} its literal plane and first tier take for {int(n[i])} weights")
    long = np.flatnonzero(extent > most)
    if long.size:
        i = int(long[0])
        raise ValueError(f"invalid radix block offsets: block {i} holds {int(extent[i])} words, more than the "
                         f"{int(most[i])} any block of {int(n[i])} weights can use")
