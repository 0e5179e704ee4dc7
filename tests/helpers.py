"""Shared builders for the parity tests: seeded bf16 bit patterns and radix
tensor dicts built by the oracle's encoder (any block size) or the
product's (1024-weight blocks)."""

from __future__ import annotations

import numpy as np

from oracle import radix_oracle as O


def finite_bits(rng: np.random.Generator, shape, spread: bool = False) -> np.ndarray:
    """Finite bf16 bits, safe under a matmul. spread=False: nine exponents
    around 2^-8 with a steep falloff (a tight tensor); spread=True: a
    geometric tail over 40 exponents, so the later tiers and the terminal
    stream carry many entries."""
    R, C = shape
    if spread:
        k = np.arange(40)
        pk = 0.75 ** k
        exps = rng.choice(100 + k, size=(R, C), p=pk / pk.sum())
    else:
        exps = rng.choice(np.arange(113, 122), size=(R, C),
                          p=np.array([.002, .003, .005, .01, .025, .055, .1, .3, .5]))
    bits = (exps.astype(np.uint16) << 7) | rng.integers(0, 128, (R, C), dtype=np.uint16)
    return bits | (rng.integers(0, 2, (R, C), dtype=np.uint16) << 15)


def escape_heavy_bits(rng: np.random.Generator, shape, escape_rate: float) -> np.ndarray:
    """Finite bits where about `escape_rate` of the weights fall outside the
    seven most common exponents (sip's tier 0), spread over 40 rarer ones."""
    R, C = shape
    common = rng.choice(np.arange(118, 125), size=(R, C))
    rare = rng.integers(70, 110, size=(R, C))
    exps = np.where(rng.random((R, C)) < escape_rate, rare, common)
    bits = (exps.astype(np.uint16) << 7) | rng.integers(0, 128, (R, C), dtype=np.uint16)
    return bits | (rng.integers(0, 2, (R, C), dtype=np.uint16) << 15)


def all_patterns(shape=(512, 513)) -> np.ndarray:
    """Every u16 pattern once, on a zero background (compressible)."""
    a = np.zeros(shape, np.uint16)
    a.flat[:65536] = np.arange(65536, dtype=np.uint16)
    return a


def oracle_dict(bits: np.ndarray, profile: str, block: int = 1024) -> dict:
    """A radix tensor dict written by the oracle's encoder."""
    p = O.pack(bits, profile, block)
    assert not p.raw, "the test tensor must ride the compressed streams"
    return pack_to_dict(p, profile)


def pack_to_dict(p: "O.Pack", profile: str) -> dict:
    stored = p.palette.nbytes + p.offsets.nbytes + p.data.nbytes
    return {"rx_palette": p.palette, "rx_offsets": p.offsets.astype(np.uint32), "rx_data": p.data.astype(np.uint32),
            "R": p.shape[0], "C": p.shape[1], "bpw": 8.0 * stored / (p.shape[0] * p.shape[1]), "codec": "radix",
            "profile": profile, "widths": list(p.widths), "block_size": p.block_size}


def dict_to_pack(d: dict) -> "O.Pack":
    return O.Pack((int(d["R"]), int(d["C"])), int(d["block_size"]), tuple(int(w) for w in d["widths"]),
                  np.asarray(d["rx_palette"], np.uint8), np.asarray(d["rx_offsets"], np.uint32),
                  np.asarray(d["rx_data"], np.uint32))


def bf16_tensor(bits: np.ndarray, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def u16_of(t) -> np.ndarray:
    import torch

    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def gemv_f64_rows(bits: np.ndarray, xf: np.ndarray, threads: int = 16):
    """The oracle's float64 dot and bound over row ranges on host threads
    (its C loop runs outside the GIL): (y, bound) float64 [M, R]."""
    from concurrent.futures import ThreadPoolExecutor

    xf = np.ascontiguousarray(np.atleast_2d(xf), dtype=np.float32)
    R = bits.shape[0]
    y = np.empty((xf.shape[0], R), np.float64)
    bound = np.empty_like(y)
    step = max(1, -(-R // (4 * threads)))

    def job(r0):
        yy, bb = O.gemv_f64(bits[r0:r0 + step], xf)
        y[:, r0:r0 + step] = yy
        bound[:, r0:r0 + step] = bb

    with ThreadPoolExecutor(threads) as ex:
        list(ex.map(job, range(0, R, step)))
    return y, bound


def gemv_f32_rows(bits: np.ndarray, xf: np.ndarray, threads: int = 16) -> np.ndarray:
    """The oracle's decode-then-matmul (fp32 accumulate) over row ranges on
    host threads: fp32 [M, R]."""
    from concurrent.futures import ThreadPoolExecutor

    xf = np.ascontiguousarray(np.atleast_2d(xf), dtype=np.float32)
    R = bits.shape[0]
    y = np.empty((xf.shape[0], R), np.float32)
    step = max(1, -(-R // (4 * threads)))

    def job(r0):
        y[:, r0:r0 + step] = O.gemv_f32(bits[r0:r0 + step], xf)

    with ThreadPoolExecutor(threads) as ex:
        list(ex.map(job, range(0, R, step)))
    return y


def planted_mistakes_rejected(y_row: np.ndarray, bits: np.ndarray, xf_row: np.ndarray, r: int) -> list:
    """The bound check's negative controls, planted in the oracle (CPU):
    for output row r of a result y_row (float, [R]) that passes the check,
    three plausible decoder or indexing mistakes must each fail it:
      - one weight's exponent off by one (bit 7 flipped) at the row's
        largest |x w| term (a wrong palette or table entry);
      - that term dropped (a lost weight);
      - the neighbouring row's sums compared (a row index off by one).
    Returns the three err/bound ratios (each must exceed 1), or None when
    the row's largest term is within twice its bound: a single term that
    small sits under the bound's absolute floor and no check of that bound
    can see it."""
    xf_row = np.asarray(xf_row, np.float32).reshape(1, -1)
    row = np.ascontiguousarray(bits[r:r + 1])
    w = O.bf16_bits_to_f32(row).astype(np.float64)
    terms = np.abs(w * xf_row.astype(np.float64))
    c = int(np.argmax(terms))
    y = float(y_row[r])
    if terms[0, c] <= 2.0 * O.gemv_f64(row, xf_row)[1][0, 0]:
        return None
    out = []
    flipped = row.copy()
    flipped[0, c] ^= np.uint16(1 << 7)
    ref, bound = O.gemv_f64(flipped, xf_row)
    out.append(abs(y - ref[0, 0]) / bound[0, 0])
    dropped = row.copy()
    dropped[0, c] &= np.uint16(0x8000)  # that weight as a signed zero: its term gone
    ref, bound = O.gemv_f64(dropped, xf_row)
    out.append(abs(y - ref[0, 0]) / bound[0, 0])
    other = r + 1 if r + 1 < bits.shape[0] else r - 1
    if other >= 0:
        ref, bound = O.gemv_f64(np.ascontiguousarray(bits[other:other + 1]), xf_row)
        out.append(abs(y - ref[0, 0]) / bound[0, 0])
    return out
