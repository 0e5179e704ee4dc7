"""The radix codec as a pack tensor: profiles, the host encoder, the raw
fallback and the descriptor gate — the producer side of the kernels'
inputs, under drinkme's function names and dict layout
(src/drinkme/codec/radix_pack.py, src/drinkme/codec/radix.py:149-238).

A radix tensor dict (src/drinkme/codec/radix_pack.py:9-22):
    rx_palette  u8  [covered]      exponents in code order, unpadded
    rx_offsets  u32 [R * NB + 1]   word directory
    rx_data     u32 [NW]           concatenated block streams
    R, C, bpw, codec = "radix", profile, widths, block_size = 1024

The codec itself runs on host threads inside libdmx_radix.so, behind
dmx_radix_native (include/dmx_radix.h), which keeps drinkme's radix_native
signature (src/drinkme/codec/radix_native.cpp:211-236). `HostCodec` binds
one tensor's geometry to that entry point's op protocol; everything in
this module that packs or unpacks goes through it.
"""

from __future__ import annotations

import ctypes as ct
from dataclasses import dataclass, field

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


def _tier_runs(widths):
    """Per nonterminal tier: (first palette entry, entries, first byte of
    its run in the device tables). A tier of width w addresses 2^w - 1
    palette entries (its last code is the escape); its run in the tables is
    those entries zero-filled up to a whole number of u32 words."""
    runs, entry, byte = [], 0, 0
    for w in tuple(widths)[:-1]:
        n = (1 << int(w)) - 1
        runs.append((entry, n, byte))
        entry += n
        byte += 4 * ((n + 4) // 4)  # == 4 * ((2^w + 2) // 4): n + 1 = 2^w, so the run always has room
    return runs


def covered_of(widths) -> int:
    """Palette entries the nonterminal tiers address."""
    return sum(n for _, n, _ in _tier_runs(widths))


def table_words(widths) -> int:
    """u32 words of the padded device tables: ((1 << w) + 2) // 4 per tier."""
    runs = _tier_runs(widths)
    return 0 if not runs else (runs[-1][2] + 4 * ((runs[-1][1] + 4) // 4)) // 4


def device_tables(palette, widths) -> np.ndarray:
    """The palette laid out as the device reads it (u8, table_words * 4
    bytes): each tier's run of entries, then zeros, so a tier's escape code
    indexes a zero byte (src/drinkme/codec/radix_pack.py:333-350)."""
    palette = np.asarray(palette, dtype=np.uint8)
    out = np.zeros(4 * table_words(widths), dtype=np.uint8)
    for entry, n, byte in _tier_runs(widths):
        out[byte:byte + n] = palette[entry:entry + n]
    return out


def palette_of_tables(tables, widths) -> np.ndarray:
    """device_tables' inverse: the unpadded palette, in code order."""
    tables = np.asarray(tables, dtype=np.uint8)
    runs = _tier_runs(widths)
    return np.concatenate([tables[b:b + n] for _, n, b in runs]).astype(np.uint8)


def block_word_bounds(n, widths):
    """(fewest, most) words a block of n weights occupies: the literal plane
    and tier 0 are fixed; later tiers and the terminal hold 0..n entries
    each (src/drinkme/codec/radix.py:149-171). `most` is also the reach
    pad the device allocation carries."""
    n = np.asarray(n, dtype=np.int64)
    words = lambda bits_each: (n * bits_each + 31) // 32  # noqa: E731
    w = [int(x) for x in widths]
    fewest = words(MANT + 1) + words(w[0])
    most = fewest
    for width in w[1:]:
        most = most + words(width)
    return fewest, most


def pad_words(widths, block: int = RADIX_BLOCK) -> int:
    return int(block_word_bounds(block, widths)[1])


def _address(a):
    return None if a is None else a.ctypes.data


@dataclass
class HostCodec:
    """One tensor's geometry bound to dmx_radix_native's op protocol.

    The library takes pointers, not lengths, so every array handed over is
    allocated here at the size the geometry implies (or its size checked
    first). One palette region covers the whole tensor: rows x
    blocks_per_row blocks, 1024 weights each, as drinkme's packs use.

    Ops: PLAN fills the tables and the directory and returns the payload's
    word count; ENCODE fills the payload; DECODE writes rows
    [first, first + count) starting at the output pointer it is given;
    CHECK_PALETTE refuses repeated, out-of-range or padding-dirty tables."""

    rows: int
    cols: int
    widths: tuple
    _w: np.ndarray = field(init=False, repr=False)

    PLAN, ENCODE, DECODE, CHECK_PALETTE = 0, 1, 2, 3

    def __post_init__(self):
        self.rows, self.cols = int(self.rows), int(self.cols)
        self.widths = tuple(int(w) for w in self.widths)
        self._w = np.array(self.widths, dtype=np.uint32)

    @property
    def blocks_per_row(self) -> int:
        return -(-self.cols // RADIX_BLOCK)

    @property
    def directory_len(self) -> int:
        return self.rows * self.blocks_per_row + 1

    def op(self, code: int, bits=None, tables=None, offsets=None, data=None, first: int = 0, count: int = 0) -> int:
        """One dmx_radix_native call; its status becomes a ValueError with
        the library's message. Returns the op's result word."""
        result = ct.c_uint64()
        err = _native.error_buffer()
        status = _native.lib().dmx_radix_native(
            code, _address(bits), self.rows, self.cols, self.rows, self.blocks_per_row, MANT, EXP,
            self._w.ctypes.data, self._w.size, _address(tables), _address(offsets), _address(data),
            0 if data is None else data.size, first, count, ct.byref(result), err, len(err))
        if status:
            raise ValueError("native radix: " + err.value.decode())
        return result.value

    def compress(self, bits: np.ndarray):
        """u16 [rows, cols] -> (device tables u8, offsets u32, data u32),
        then decoded back and compared: a stream that does not reproduce
        its source is never returned."""
        tables = np.zeros(4 * table_words(self.widths), dtype=np.uint8)
        offsets = np.zeros(self.directory_len, dtype=np.uint32)
        data = np.zeros(self.op(self.PLAN, bits, tables, offsets), dtype=np.uint32)
        self.op(self.ENCODE, bits, tables, offsets, data)
        if not np.array_equal(self.expand(tables, offsets, data), bits):
            raise ValueError("native radix: CPU round trip differs from the source bits")
        return tables, offsets, data

    def expand(self, tables, offsets, data, out=None, first: int = 0, count: int | None = None) -> np.ndarray:
        """Rows [first, first + count) of the tensor into out[first:] (a new
        u16 [rows, cols] array when out is None)."""
        if out is None:
            out = np.empty((self.rows, self.cols), dtype=np.uint16)
        count = self.rows - first if count is None else count
        self.op(self.DECODE, out[first:], tables, offsets, data, first, count)
        return out


def encode(U: np.ndarray, widths):
    """u16 [R, C] bf16 bits -> (palette u8 unpadded, offsets u32, data u32),
    1024-weight blocks, one palette per tensor; verified by decoding back."""
    U = np.ascontiguousarray(U, dtype=np.uint16)
    tables, offsets, data = HostCodec(*U.shape, widths).compress(U)
    return palette_of_tables(tables, widths), offsets, data


def decode(palette, offsets, data, R: int, C: int, widths) -> np.ndarray:
    """The host decoder (dmx_radix_native op 2): u16 [R, C]."""
    codec = HostCodec(R, C, widths)
    if offsets.ndim != 1 or offsets.size != codec.directory_len:
        raise ValueError("native radix: invalid radix block offsets")
    if palette.ndim != 1 or palette.size != covered_of(widths):
        raise ValueError("native radix: invalid radix palette entries")
    return codec.expand(device_tables(palette, widths), np.ascontiguousarray(offsets, dtype=np.uint32),
                        np.ascontiguousarray(data, dtype=np.uint32))


def _bit_plane(U, who: str) -> np.ndarray:
    U = np.ascontiguousarray(U, dtype=np.uint16)
    if U.ndim != 2 or 0 in U.shape:
        raise ValueError(f"{who}: need a nonempty 2D uint16 array")
    return U


def footprint(palette, offsets, data, widths) -> tuple:
    """(stored, device) bytes of a radix tensor: the three arrays as the
    pack stores them, and as the device holds them (the palette as padded
    tables, the reach pad excluded). drinkme stores a tensor raw when either
    reaches the raw plane's 2 bytes per weight (src/drinkme/codec/
    radix_pack.py:166-172)."""
    body = offsets.nbytes + data.nbytes
    return body + palette.nbytes, body + 4 * table_words(widths)


def pack_array_radix(U: np.ndarray, compression_profile: str) -> dict | None:
    """u16 [R, C] bf16 bits -> the radix tensor dict, or None when radix
    would not compress it (the caller stores it raw)
    (src/drinkme/codec/radix_pack.py:175-205)."""
    U = _bit_plane(U, "pack_array_radix")
    widths = widths_of(compression_profile)
    arrays = dict(zip(ARRAYS_RADIX, encode(U, widths)))
    stored, device = footprint(*arrays.values(), widths)
    if max(stored, device) >= U.nbytes:
        return None
    R, C = U.shape
    arrays.update(R=R, C=C, bpw=8.0 * stored / U.size, codec=RADIX, profile=compression_profile,
                  widths=list(widths), block_size=RADIX_BLOCK)
    return arrays


def raw_dict(U: np.ndarray) -> dict:
    """The raw fallback tensor: the bf16 bit patterns verbatim."""
    U = _bit_plane(U, "raw_dict")
    return dict(raw_bits=U, R=U.shape[0], C=U.shape[1], bpw=16.0, codec=RAW)


def pack_weight_radix(U: np.ndarray, compression_profile: str) -> dict:
    """One tensor: the radix dict, or the raw dict when radix would expand
    it (src/drinkme/codec/radix_pack.py:217-236, over u16 bits)."""
    return pack_array_radix(U, compression_profile) or raw_dict(U)


def padded_palette_words(palette: np.ndarray, widths) -> np.ndarray:
    """device_tables as u32 words, the runtime dict's rx_palette."""
    return device_tables(palette, widths).view(np.uint32)


# ---------------------------------------------------------------------------
# The descriptor gate (src/drinkme/codec/radix.py:174-238): a tensor is
# refused before any device allocation unless its geometry, palette and
# directory are consistent. The gate proves every block's extent lies
# between its fixed streams and the widest block of its weight count; that
# is what bounds the device readers' reach (the allocation's pad). Each
# stage below returns the first fault it finds, or None, with the message
# drinkme's callers and tests match on.


def _widths_fault(d):
    w = d.widths
    if not 2 <= len(w) <= 8 or w[-1] != EXP or min(w) < 1 or max(w) > 8:
        return "radix needs 2..8 widths in 1..8, ending with the exponent width"
    if covered_of(w) > 1 << EXP:
        return "radix tiers exceed the exponent alphabet"
    return None


def _geometry_fault(d):
    B = d.block
    if not 32 <= B <= 4096 or B & (B - 1):
        return "invalid radix block size"
    if d.R <= 0 or d.C <= 0:
        return "invalid radix shape"
    return None


def _array_fault(d):
    kinds = ((d.palette, np.uint8, "invalid radix palette"), (d.offsets, np.uint32, "invalid radix directory"))
    for a, dtype, message in kinds:
        if a.ndim != 1 or a.dtype != dtype:
            return message
    if d.palette.size != covered_of(d.widths) or np.unique(d.palette).size != d.palette.size:
        return "invalid radix palette entries"
    if d.data.ndim != 1 or d.data.dtype != np.uint32:
        return "invalid radix payload"
    return None


def _directory_fault(d):
    o = d.offsets
    if o.size != d.R * d.blocks_per_row + 1 or o[0] != 0 or int(o[-1]) != d.data.size:
        return "invalid radix block offsets"
    extent = np.diff(o.astype(np.int64))
    if extent.size and extent.min() <= 0:
        return "invalid radix block offsets"
    # weights per block: full blocks, the row's last holds the remainder
    per_row = np.full(d.blocks_per_row, d.block, dtype=np.int64)
    per_row[-1] = d.C - d.block * (d.blocks_per_row - 1)
    n = np.tile(per_row, d.R)
    fewest, most = block_word_bounds(n, d.widths)
    for bad, limit, text in ((extent < fewest, fewest, "word(s), fewer than the {lim} its literal plane and first "
                              "tier take for {n} weights"),
                             (extent > most, most, "words, more than the {lim} any block of {n} weights can use")):
        hits = np.flatnonzero(bad)
        if hits.size:
            i = int(hits[0])
            return (f"invalid radix block offsets: block {i} holds {int(extent[i])} "
                    + text.format(lim=int(limit[i]), n=int(n[i])))
    return None


@dataclass
class _Descriptor:
    widths: tuple
    block: int
    R: int
    C: int
    palette: np.ndarray
    offsets: np.ndarray
    data: np.ndarray

    @property
    def blocks_per_row(self) -> int:
        return -(-self.C // self.block)


_GATE = (_widths_fault, _geometry_fault, _array_fault, _directory_fault)


def validate_radix(p: dict) -> None:
    """Raises ValueError naming the first fault of the radix dict `p`:
    widths, block size and shape, array types and palette entries, then
    the directory (0 to the payload end, strictly increasing, every block's
    extent within its bounds)."""
    d = _Descriptor(tuple(int(w) for w in p["widths"]), int(p["block_size"]), int(p["R"]), int(p["C"]),
                    np.asarray(p["rx_palette"]), np.asarray(p["rx_offsets"]), np.asarray(p["rx_data"]))
    for stage in _GATE:
        fault = stage(d)
        if fault:
            raise ValueError(fault)
