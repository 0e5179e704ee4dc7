"""Writes the golden vectors the oracle and the product codec are pinned to.

    make -C oracle ref && python tests/golden/make_golden.py

Every vector is encoded by drinkme's own C++ codec, compiled from its source
file by `make -C oracle ref` (oracle/_ref/libradix_native_ref.so), on inputs
this script generates from fixed seeds:

  golden.json   per case and profile: shape, palette bytes, payload word
                count and the SHA-256 of the palette, directory and payload
                arrays the drinkme encoder wrote, plus the SHA-256 of the
                source bits
  small.npz     the full arrays (source bits, palette, offsets, data) of
                one small ragged case at every profile

Inputs: bf16 bits from drinkme_amd.synth (counter-based, N(0, 0.02) and
Student-t), from numpy's PCG64 (a spread of exponents, ragged widths) and
the 65,536-pattern tensor on a zero background.
"""

from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from drinkme_amd import synth  # noqa: E402
from oracle import radix_oracle as O  # noqa: E402

PROFILES = {"sip": (3, 8), "balanced": (2, 3, 8), "gulp": (2, 2, 4, 8)}


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def spread_bits(seed: int, shape) -> np.ndarray:
    """A geometric tail over 40 exponents (many escapes), random signs and
    mantissas."""
    rng = np.random.default_rng(seed)
    k = np.arange(40)
    pk = 0.7 ** k
    exps = rng.choice(95 + k, size=shape, p=pk / pk.sum()).astype(np.uint16)
    bits = (exps << 7) | rng.integers(0, 128, shape, dtype=np.uint16)
    return bits | (rng.integers(0, 2, shape, dtype=np.uint16) << 15)


def all_patterns() -> np.ndarray:
    a = np.zeros((512, 513), np.uint16)
    a.flat[:65536] = np.arange(65536, dtype=np.uint16)
    return a


def cases():
    yield "linear_4096x4096_normal", synth.weight("c1", 0, "w", 4096, 4096), ("sip", "gulp")
    yield "gate_1024x4096_normal", synth.weight("qwen3-8b", 0, "gate", 1024, 4096), ("sip", "balanced", "gulp")
    yield "down_512x12288_normal", synth.weight("qwen3-8b", 0, "down", 512, 12288), ("sip", "gulp")
    yield "t4_512x5120", synth.weight("c5", 0, "q", 512, 5120, synth.STUDENT_T4), ("sip", "gulp")
    yield "spread_96x2050", spread_bits(11, (96, 2050)), ("sip", "balanced", "gulp")
    yield "spread_7x33", spread_bits(12, (7, 33)), ("sip", "balanced", "gulp")
    yield "all_patterns_512x513", all_patterns(), ("sip", "balanced", "gulp")


def main() -> None:
    if not O.ref_available():
        raise SystemExit("the compiled drinkme codec is missing: run `make -C oracle ref`")
    out = {"encoder": "drinkme src/drinkme/codec/radix_native.cpp (plan + encode), compiled by oracle/Makefile",
           "cases": {}}
    small = {}
    for name, bits, profiles in cases():
        entry = {"shape": list(bits.shape), "source_sha256": sha(bits), "profiles": {}}
        for prof in profiles:
            pal, off, data = O.ref_encode(bits, PROFILES[prof])
            back = O.ref_decode(pal, off, data, bits.shape[0], bits.shape[1], PROFILES[prof])
            assert np.array_equal(back, bits), (name, prof)
            entry["profiles"][prof] = {"palette": pal.tolist(), "words": int(data.size),
                                       "palette_sha256": sha(pal), "offsets_sha256": sha(off),
                                       "data_sha256": sha(data)}
            if name == "spread_96x2050":
                small[f"{prof}_palette"] = pal
                small[f"{prof}_offsets"] = off
                small[f"{prof}_data"] = data
        if name == "spread_96x2050":
            small["bits"] = bits
        out["cases"][name] = entry
        print(name, {p: e["words"] for p, e in entry["profiles"].items()}, flush=True)
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(out, f, indent=1)
    np.savez_compressed(os.path.join(HERE, "small.npz"), **small)


if __name__ == "__main__":
    main()
