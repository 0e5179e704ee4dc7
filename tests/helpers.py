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
