"""The operator surface over the HIP arms: drinkme's runtime dict
(to_device_radix, src/drinkme/codec/swap.py:80-161) and the resident
compressed Linear with its M router and single-rounding epilogue
(CompressedLinear / RadixCompressedLinear, src/drinkme/codec/swap.py:
228-456).

Routes (src/drinkme/codec/swap.py:302-335):
  M == 1          "gemv"   fused decode + GEMV, bias in fp32, one rounding
  2 <= M <= 8     "mc"     the same kernel family over M activation rows
  M >= 9          "dense"  decode the weight once (transient) + F.linear
  M > 8, dense
  disabled        "loop"   one M = 1 GEMV per row
There is no CPU route: the arms run on the GPU and a CPU tensor is refused.
"""

from __future__ import annotations

import os
import warnings

import numpy as np
import torch

from . import radix_ops
from .radix_pack import ARRAYS_RADIX, block_word_bounds, padded_palette_words, validate_radix

FORMAT_VERSION = 1
GEMM_MIN_ROWS = radix_ops.MC_MAX + 1  # src/drinkme/codec/swap.py:251

_DENSE_MIN: int | None = None


def _dense_min() -> int:
    """DRINKME_PREFILL_DENSE_MIN if set (<= 0 disables the dense arm), else
    GEMM_MIN_ROWS; read once (src/drinkme/codec/swap.py:208-225)."""
    global _DENSE_MIN
    if _DENSE_MIN is None:
        raw = os.environ.get("DRINKME_PREFILL_DENSE_MIN", "").strip()
        try:
            _DENSE_MIN = int(raw) if raw else GEMM_MIN_ROWS
        except ValueError:
            warnings.warn(f"DRINKME_PREFILL_DENSE_MIN={raw!r} is not an integer; using {GEMM_MIN_ROWS}")
            _DENSE_MIN = GEMM_MIN_ROWS
    return _DENSE_MIN


def to_device_radix(pack: dict, device="cuda") -> dict:
    """A radix tensor dict -> device-resident runtime buffers
    (src/drinkme/codec/swap.py:80-161):

      rx_data      u32 [NW + pad]  the block streams, then `pad` zero words
                                   (block_word_bounds(B)[1]: sip 608, gulp 768)
      rx_offsets   u32 [NBK + 1]   the word directory
      rx_palette   u32 [...]       the padded per-tier lookup tables
      rx_schedule  u16 [NBK]       > 2 tiers: the per-block tier stream
                                   lengths, prepared on the device; else empty
    The descriptors pass the gate (validate_radix) before any allocation."""
    validate_radix(pack)
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError("to_device_radix: the radix arms run on the GPU")
    R, C = int(pack["R"]), int(pack["C"])
    widths = tuple(int(w) for w in pack["widths"])
    B = int(pack["block_size"])
    nblk = R * ((C + B - 1) // B)
    payload = np.ascontiguousarray(pack["rx_data"], dtype=np.uint32).reshape(-1)
    pad = int(block_word_bounds(B, widths)[1])
    data = torch.zeros(payload.size + pad, dtype=torch.uint32, device=dev)
    data[: payload.size].copy_(torch.from_numpy(payload))
    offsets = torch.from_numpy(np.ascontiguousarray(pack["rx_offsets"], dtype=np.uint32)).to(dev)
    palette = torch.from_numpy(padded_palette_words(pack["rx_palette"], widths).copy()).to(dev)
    if len(widths) > 2:
        schedule = radix_ops.prepare_schedule(data, offsets, C, widths, B, nblk)
    else:
        schedule = torch.empty(0, dtype=torch.uint16, device=dev)
    return {
        **{k: v for k, v in pack.items() if k not in ARRAYS_RADIX},
        "rx_data": data,
        "rx_offsets": offsets,
        "rx_palette": palette,
        "rx_schedule": schedule,
        "rx_palette_np": np.ascontiguousarray(pack["rx_palette"], dtype=np.uint8),
        "NW": int(payload.size), "rx_pad_words": pad,
        "R": R, "C": C, "widths": widths, "block_size": B, "NBK": nblk,
        "codec": "radix", "format_version": FORMAT_VERSION, "layout": 0,
    }


def resident_bytes(p: dict) -> int:
    """Device bytes of a runtime dict: payload + pad, directory, tables,
    schedule."""
    return sum(p[k].numel() * p[k].element_size() for k in ("rx_data", "rx_offsets", "rx_palette", "rx_schedule"))


class RadixCompressedLinear(torch.nn.Module):
    """A radix-coded Linear resident on the GPU: the M router, the arms and
    the fp32-accumulate-then-round-once epilogue of drinkme's
    RadixCompressedLinear (src/drinkme/codec/swap.py:384-456)."""

    GEMM_MIN_ROWS = GEMM_MIN_ROWS

    def __init__(self, runtime: dict, bias=None):
        super().__init__()
        if runtime.get("codec") != "radix":
            raise ValueError("RadixCompressedLinear needs a to_device_radix runtime dict")
        self.p = runtime
        self.bias = bias
        self.R, self.C = int(runtime["R"]), int(runtime["C"])
        self.tensor_codec = "radix"
        self.layout = 0

    def _route(self, x) -> str:
        if x.device.type == "cpu":
            return "cpu"
        return self._route_rows(x.numel() // x.shape[-1])

    @staticmethod
    def _route_rows(m: int) -> str:
        if m == 1:
            return "gemv"
        dense_min = _dense_min()
        if 0 < dense_min <= m:
            return "dense"
        if m <= radix_ops.MC_MAX:
            return "mc"
        return "loop"

    def forward(self, x):
        return self._forward(x, self._route(x))

    def _forward(self, x, route: str):
        if route == "cpu":
            raise RuntimeError("RadixCompressedLinear: the radix arms run on the GPU; x is on the CPU")
        shape = x.shape
        xf = x.reshape(-1, self.C)
        if route in ("gemv", "mc") and x.dtype in (torch.bfloat16, torch.float32):
            # one launch: fp32 accumulation, the bias in fp32, one rounding to x.dtype
            out = radix_ops.gemv_rows(self.p, xf, self.bias, x.dtype)
            return out.reshape(*shape[:-1], self.R)
        if route == "dense":
            W = radix_ops.decode_weight(self.p)
            out = torch.nn.functional.linear(xf.to(W.dtype) if xf.dtype != W.dtype else xf, W, self.bias)
            return out.to(x.dtype).reshape(*shape[:-1], self.R)
        # other dtypes through fp32 rows, or the per-row loop
        rows = xf.shape[0]
        outs = torch.empty(rows, self.R, device=x.device, dtype=torch.float32)
        step = 1 if route == "loop" else rows
        for i in range(0, rows, step):
            outs[i:i + step] = radix_ops.gemv_rows(self.p, xf[i:i + step].float(), None, torch.float32)
        if self.bias is not None:
            outs = outs + self.bias
        return outs.to(x.dtype).reshape(*shape[:-1], self.R)


def make_module(pack: dict, bias=None, device="cuda") -> torch.nn.Module:
    """The served module for one packed tensor: RadixCompressedLinear over
    its runtime dict (src/drinkme/codec/swap.py:900-919, radix only)."""
    if pack.get("codec") != "radix":
        raise ValueError("make_module: not a radix tensor dict")
    return RadixCompressedLinear(to_device_radix(pack, device), bias)
