"""Seeded synthetic weights and activations for the benchmark workloads.

Every tensor is its own counter-based stream (dmx_synth_bf16), keyed by
(workload, layer, tensor name): the same bits on any machine and at any
thread count. Weights are N(0, 0.02) — or Student-t(nu = 4) scaled to
std 0.02 for the 32B-class stack — drawn in float64, rounded to float32,
then to bf16 (nearest even); activations are N(0, 1) bf16.
"""

from __future__ import annotations

import hashlib

import numpy as np

from . import _native

SEED = 20260501
NORMAL, STUDENT_T4 = 0, 1

# Qwen3-8B decoder layer: (name, rows, cols)
QWEN3_8B_LAYER = (("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
                  ("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288))
QWEN3_8B_LAYERS = 36
QWEN3_8B_LM_HEAD = ("lm_head", 151936, 4096)

# 32B-class stack (hidden 5120, 64 layers)
CLASS_32B_LAYER = (("q", 8192, 5120), ("k", 1024, 5120), ("v", 1024, 5120), ("o", 5120, 8192),
                   ("gate", 25600, 5120), ("up", 25600, 5120), ("down", 5120, 25600))
CLASS_32B_LAYERS = 64


def stream_id(*key) -> int:
    """A 64-bit stream id for a (workload, layer, tensor) key."""
    h = hashlib.sha256("/".join(str(k) for k in key).encode()).digest()
    return int.from_bytes(h[:8], "little")


def bf16_bits(key: tuple, shape, scale: float = 0.02, dist: int = NORMAL, seed: int = SEED) -> np.ndarray:
    """u16 bf16 bit patterns of the given shape for stream `key`."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.uint16)
    err = _native.error_buffer()
    st = _native.lib().dmx_synth_bf16(seed, stream_id(*key), n, float(scale), dist, out.ctypes.data, err, len(err))
    _native.check(st, err, "dmx_synth_bf16")
    return out.reshape(shape)


def weight(workload: str, layer, name: str, rows: int, cols: int, dist: int = NORMAL) -> np.ndarray:
    return bf16_bits((workload, layer, name), (rows, cols), 0.02, dist)


def activation(workload: str, name: str, m: int, cols: int) -> np.ndarray:
    return bf16_bits((workload, "x", name), (m, cols), 1.0, NORMAL)


def qwen3_8b_step():
    """The (layer, name, rows, cols) list of one Qwen3-8B decode step's
    compressed Linears, in execution order: 36 layers then lm_head."""
    items = [(layer, name, r, c) for layer in range(QWEN3_8B_LAYERS) for name, r, c in QWEN3_8B_LAYER]
    items.append(("head",) + QWEN3_8B_LM_HEAD)
    return items
