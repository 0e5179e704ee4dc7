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

Beside it, the raw bf16 surface that binds the same ops module:
NarrowLinear / install_narrow (src/drinkme/codec/swap.py:530-627), the
Linears under the codec's row threshold, through radix_ops.gemv_narrow;
and to_device_twin (swap.py:168-196), a raw bf16 weight's dict that the
GEMV calls run through the raw kernel.
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


def eligible(child) -> bool:
    """A Linear the codec takes (src/drinkme/codec/swap.py:850-854): bf16,
    C % 4 == 0, both dims >= 1024."""
    if not isinstance(child, torch.nn.Linear):
        return False
    w = child.weight.data
    return w.dtype == torch.bfloat16 and w.shape[1] % 4 == 0 and min(w.shape) >= 1024


class NarrowLinear(torch.nn.Linear):
    """A raw bf16 Linear under the codec's row threshold, served by the raw
    GEMV (src/drinkme/codec/swap.py:530-610): M <= 8 rows in one launch of
    radix_ops.gemv_narrow (fp32 accumulate, the bias added in fp32, one
    rounding); more rows, or a CPU tensor, is F.linear. The weight and bias
    are the adopted Linear's own Parameters. Row m of an M-row call is the
    one-row call bit for bit."""

    BLOCK = 512  # drinkme's launch knobs, passed through (swap.py:577-578)
    NUM_WARPS = 4
    MAX_ROWS = 1024  # swap.py:581-582
    MIN_COLS = 1024

    @classmethod
    def wants(cls, mod) -> bool:
        if type(mod) is not torch.nn.Linear or eligible(mod):
            return False
        w = mod.weight
        return (w.dtype == torch.bfloat16 and w.device.type == "cuda" and w.shape[0] <= cls.MAX_ROWS
                and w.shape[1] >= cls.MIN_COLS and w.shape[1] % 4 == 0)

    @classmethod
    def adopt(cls, lin: torch.nn.Linear) -> "NarrowLinear":
        """The same parameters under this class: no copy."""
        new = cls(lin.in_features, lin.out_features, bias=lin.bias is not None, device="meta")
        new.weight = lin.weight
        new.bias = lin.bias
        return new

    def forward(self, x):
        shape = x.shape
        xm = x.reshape(-1, self.in_features)
        if xm.shape[0] > radix_ops.MC_MAX or x.device.type != "cuda":
            return torch.nn.functional.linear(x, self.weight, self.bias)
        y = radix_ops.gemv_narrow(self.weight, xm, self.bias, self.BLOCK, self.NUM_WARPS)
        return y.reshape(*shape[:-1], self.out_features)


def install_narrow(model, device: str) -> list:
    """Every raw Linear NarrowLinear.wants, adopted in place; returns the
    (name, (R, C)) list (src/drinkme/codec/swap.py:613-627). Nothing off
    the GPU."""
    if not str(device).startswith("cuda"):
        return []
    done = []
    for parent_name, parent in list(model.named_modules()):
        for child_name, child in list(parent.named_children()):
            if NarrowLinear.wants(child):
                setattr(parent, child_name, NarrowLinear.adopt(child))
                name = f"{parent_name}.{child_name}" if parent_name else child_name
                done.append((name, tuple(child.weight.shape)))
    return done


def to_device_twin(w_bf16, widths=(3, 8), device: str = "cuda") -> dict:
    """A raw bf16 weight [R, C] as a twin dict (src/drinkme/codec/swap.py:
    168-196): the weight resident and row-major, codec "twin". The GEMV
    calls of radix_ops run it through the raw kernel."""
    w = w_bf16.detach()
    if w.dtype != torch.bfloat16:
        raise TypeError(f"to_device_twin: {w.dtype} is not bf16")
    R, C = int(w.shape[0]), int(w.shape[1])
    B = 1024
    return {"weight": w.contiguous().to(torch.device(device)), "R": R, "C": C,
            "widths": tuple(int(x) for x in widths), "block_size": B, "NBK": R * ((C + B - 1) // B),
            "codec": "twin", "layout": 0}
