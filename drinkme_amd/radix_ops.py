"""drinkme's radix_ops surface (src/drinkme/codec/radix_ops.py:341-441) over
libdmx_radix.so: the same functions, arguments and results, so the module
seam that binds radix_ops (src/drinkme/codec/swap.py:60-65) can bind this
module instead.

  gemv_fused(p, x, bias, out_dtype)  x [C] -> [1, R], bias in fp32, one rounding
  gemv(p, x)                         x [C] -> fp32 [R], no bias
  gemv_mc(p, x)                      x [M, C], 1 <= M <= 8 -> fp32 [M, R]
  gemv_rows(p, x, bias, out_dtype)   x [M, C] -> [M, R], bias and one rounding
                                     fused (the mc arm plus swap's epilogue)
  gemv_narrow(w, x, bias, ...)       raw bf16 w [R, C], x [M, C] -> [M, R] in x's dtype
  decode_bits(p)                     -> u16 [R, C], the source bit patterns
  decode_weight(p)                   -> bf16 [R, C]
  prepare_schedule(...)              -> u16 [nblocks], the gulp stream lengths
  read_bytes(p)                      bytes one call streams

`p` is a runtime dict from swap.to_device_radix, or a twin dict (codec
"twin", swap.to_device_twin's: the raw bf16 `weight` [R, C]), which the
GEMV calls run through the raw kernel (drinkme's RAW=True route,
radix_ops.py:252-255). Every call launches on torch's current stream and
allocates only its output, with torch.
"""

from __future__ import annotations

import ctypes as ct
import threading

import torch

from . import _native

MC_MAX = 8  # src/drinkme/codec/ops.py:19

_DTYPE = {torch.bfloat16: _native.DMX_BF16, torch.float32: _native.DMX_F32}


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device=None):
    """The handle of torch's current stream on `device` (torch's current
    device when None). torch's raw-handle accessor costs well under a
    microsecond; torch.cuda.current_stream() builds a Stream object (about
    3 us a call), which this falls back to only where the accessor is
    missing."""
    if _raw_stream is not None:
        index = device.index if device is not None and device.index is not None else torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


def descriptor(p: dict) -> _native.RadixTensor:
    """The dmx_radix_tensor of a runtime dict, kept in the dict with the
    buffer addresses and sizes it was built from: a copy of the dict with
    another buffer in it (dict(p, rx_data=...)) gets a descriptor of its
    own."""
    sched = p.get("rx_schedule")
    key = (p["rx_data"].data_ptr(), p["rx_offsets"].data_ptr(), p["rx_palette"].data_ptr(),
           sched.data_ptr() if sched is not None and sched.numel() else 0, int(p["NW"]), int(p["rx_pad_words"]),
           int(p["R"]), int(p["C"]), int(p["block_size"]), tuple(int(w) for w in p["widths"]))
    cached = p.get("_dmx")
    t = cached[1] if cached is not None and cached[0] == key else None
    if t is None:
        widths = [int(w) for w in p["widths"]]
        t = _native.RadixTensor()
        t.data = p["rx_data"].data_ptr()
        t.offsets = p["rx_offsets"].data_ptr()
        t.palette = p["rx_palette"].data_ptr()
        t.schedule = sched.data_ptr() if sched is not None and sched.numel() else None
        t.payload_words = int(p["NW"])
        t.pad_words = int(p["rx_pad_words"])
        t.rows, t.cols, t.block_size = int(p["R"]), int(p["C"]), int(p["block_size"])
        t.n_widths = len(widths)
        for i, w in enumerate(widths):
            t.widths[i] = w
        p["_dmx"] = (key, t)
    return t


_tls = threading.local()


def _error_buffer():
    """This thread's error buffer for the launchers below (the library
    writes into it only when a call fails)."""
    buf = getattr(_tls, "err", None)
    if buf is None:
        buf = _tls.err = _native.error_buffer()
    return buf


def _buffers(p: dict) -> tuple:
    """The addresses of a runtime dict's buffers: a launcher's descriptor is
    rebuilt when any of them moves (another tensor in the dict, or new
    storage under the same tensor)."""
    sched = p.get("rx_schedule")
    return (p["rx_data"].data_ptr(), p["rx_offsets"].data_ptr(), p["rx_palette"].data_ptr(),
            sched.data_ptr() if sched is not None else 0)


def _dtype_code(dtype, what):
    if dtype not in _DTYPE:
        raise TypeError(f"{what}: {dtype} is not bf16 or fp32")
    return _DTYPE[dtype]


def _is_twin(p: dict) -> bool:
    """A twin dict: the raw bf16 weight, run by the compressed tensor's own
    kernel with the decode replaced by a raw load (radix_ops.py:252-255)."""
    return p.get("codec") == "twin"


def _check_rows(x, C, device, bias, R, what):
    if x.dim() != 2 or x.shape[1] != C:
        raise ValueError(f"{what}: x must be [M, {C}], got {tuple(x.shape)}")
    M = x.shape[0]
    if not 1 <= M <= MC_MAX:
        raise ValueError(f"{what}: M={M} outside 1..{MC_MAX}")
    if x.device != device:
        raise ValueError(f"{what}: x is not on the weight's device")
    if bias is not None and (bias.numel() != R or bias.device != x.device):
        raise ValueError(f"{what}: bias must hold R elements on the weight's device")
    return M


def _raw_rows(w: torch.Tensor, x: torch.Tensor, bias, out_dtype, what: str) -> torch.Tensor:
    """The raw bf16 GEMV (dmx_gemv_narrow): w [R, C] bf16, x [M, C]."""
    if w.dim() != 2 or w.dtype != torch.bfloat16:
        raise TypeError(f"{what}: the weight must be a 2-D bf16 tensor, got {w.dtype} {tuple(w.shape)}")
    R, C = int(w.shape[0]), int(w.shape[1])
    M = _check_rows(x, C, w.device, bias, R, what)
    w, x = w.contiguous(), x.contiguous()
    out = torch.empty((M, R), dtype=out_dtype, device=x.device)
    xd = _dtype_code(x.dtype, "activation")
    od = _dtype_code(out_dtype, "output")
    bias = bias.contiguous() if bias is not None else None
    bd = _dtype_code(bias.dtype, "bias") if bias is not None else 0
    err = _native.error_buffer()
    st = _native.lib().dmx_gemv_narrow(w.data_ptr(), R, C, x.data_ptr(), xd, M,
                                       bias.data_ptr() if bias is not None else None, bd, out.data_ptr(), od,
                                       _stream(x.device), err, len(err))
    _native.check(st, err, "dmx_gemv_narrow")
    return out


def _twin_rows(p: dict, x: torch.Tensor, bias, out_dtype) -> torch.Tensor:
    """A twin dict's GEMV (dmx_radix_gemv_twin): the kernel its compressed
    tensor runs (the dict's widths and block size), reading the raw weight in
    place of the decode (radix_kernel_gpu.py:639-668), so its sums are the
    compressed tensor's bit for bit."""
    w = p["weight"]
    if w.dim() != 2 or w.dtype != torch.bfloat16:
        raise TypeError(f"raw gemv: the weight must be a 2-D bf16 tensor, got {w.dtype} {tuple(w.shape)}")
    R, C = int(w.shape[0]), int(w.shape[1])
    M = _check_rows(x, C, w.device, bias, R, "raw gemv")
    w, x = w.contiguous(), x.contiguous()
    out = torch.empty((M, R), dtype=out_dtype, device=x.device)
    xd = _dtype_code(x.dtype, "activation")
    od = _dtype_code(out_dtype, "output")
    bias = bias.contiguous() if bias is not None else None
    bd = _dtype_code(bias.dtype, "bias") if bias is not None else 0
    widths = [int(v) for v in p.get("widths", (3, 8))]
    warr = (ct.c_uint32 * len(widths))(*widths)
    err = _native.error_buffer()
    st = _native.lib().dmx_radix_gemv_twin(w.data_ptr(), R, C, int(p.get("block_size", 1024)), len(widths), warr,
                                           x.data_ptr(), xd, M, bias.data_ptr() if bias is not None else None, bd,
                                           out.data_ptr(), od, _stream(x.device), err, len(err))
    _native.check(st, err, "dmx_radix_gemv_twin")
    return out


def gemv_rows(p: dict, x: torch.Tensor, bias=None, out_dtype=torch.float32) -> torch.Tensor:
    """x [M, C] (bf16 or fp32, 1 <= M <= 8) -> [M, R] in out_dtype: the rows
    accumulated in fp32, the bias (bf16 or fp32, or None) added in fp32,
    one rounding."""
    if _is_twin(p):
        return _twin_rows(p, x, bias, out_dtype)
    R = int(p["R"])
    dev = p["rx_data"].device
    M = _check_rows(x, int(p["C"]), dev, bias, R, "radix gemv")
    if not x.is_contiguous():
        x = x.contiguous()
    out = torch.empty((M, R), dtype=out_dtype, device=dev)
    xd = _dtype_code(x.dtype, "activation")
    od = _dtype_code(out_dtype, "output")
    if bias is not None:
        bias = bias.contiguous()
        bd = _dtype_code(bias.dtype, "bias")
    else:
        bd = 0
    err = _native.error_buffer()
    st = _native.lib().dmx_radix_gemv(ct.byref(descriptor(p)), x.data_ptr(), xd, M,
                                       bias.data_ptr() if bias is not None else None, bd, out.data_ptr(), od,
                                       _stream(dev), err, len(err))
    _native.check(st, err, "dmx_radix_gemv")
    return out


def _leading_rows(x: torch.Tensor, C: int, device, what: str) -> int:
    """M, the rows of x [..., C] (the product of its leading dimensions),
    after the checks every launcher makes."""
    if x.dim() == 0 or x.shape[-1] != C:
        raise ValueError(f"{what}: x must be [..., {C}], got {tuple(x.shape)}")
    M = x.numel() // C
    if not 1 <= M <= MC_MAX:
        raise ValueError(f"{what}: M={M} outside 1..{MC_MAX}")
    if x.device != device:
        raise ValueError(f"{what}: x is not on the weight's device")
    return M


class RowsLauncher:
    """dmx_radix_gemv for one radix tensor that a caller (a module) launches
    again and again: its descriptor is built once, and again only when the
    runtime dict holds other buffers than at the last call. call(x, bias,
    out_dtype): x [..., C] (bf16 or fp32; M, the product of the leading
    dimensions, in 1..MC_MAX) -> [..., R] in out_dtype, gemv_rows' result
    bit for bit."""

    def __init__(self, p: dict):
        if _is_twin(p):
            raise ValueError("RowsLauncher: a radix runtime dict, not a twin")
        self.p = p
        self.R, self.C = int(p["R"]), int(p["C"])
        self.device = p["rx_data"].device
        self._held = None

    def _pointer(self):
        held = _buffers(self.p)
        if held != self._held:
            self._ptr = ct.pointer(descriptor(self.p))
            self._held = held
        return self._ptr

    def __call__(self, x: torch.Tensor, bias=None, out_dtype=torch.float32) -> torch.Tensor:
        M = _leading_rows(x, self.C, self.device, "radix gemv")
        if not x.is_contiguous():
            x = x.contiguous()
        xd = _dtype_code(x.dtype, "activation")
        od = _dtype_code(out_dtype, "output")
        bd = 0
        if bias is not None:
            if bias.numel() != self.R or bias.device != x.device:
                raise ValueError("radix gemv: bias must hold R elements on the weight's device")
            bias = bias.contiguous()
            bd = _dtype_code(bias.dtype, "bias")
        out = torch.empty((*x.shape[:-1], self.R), dtype=out_dtype, device=self.device)
        err = _error_buffer()
        st = _native.lib().dmx_radix_gemv(self._pointer(), x.data_ptr(), xd, M,
                                           bias.data_ptr() if bias is not None else None, bd, out.data_ptr(), od,
                                           _stream(self.device), err, len(err))
        _native.check(st, err, "dmx_radix_gemv")
        return out


def gemv_narrow(w: torch.Tensor, x: torch.Tensor, bias, block: int = 512, num_warps: int = 4) -> torch.Tensor:
    """swap.NarrowLinear's forward for 1 <= M <= 8 rows (radix_ops.py:
    401-415): x [M, C] (bf16 or fp32) against the row-major bf16 weight
    w [R, C] -> [M, R] in x's dtype, the bias (if any) added in fp32 before
    the one rounding. Raises ValueError for M outside 1..8. `block` and
    `num_warps` are accepted for the signature and ignored: the launch
    shape is the library's."""
    del block, num_warps
    return _raw_rows(w, x, bias, x.dtype, "gemv_narrow")


def gemv_fused(p: dict, x: torch.Tensor, bias, out_dtype=torch.bfloat16) -> torch.Tensor:
    """The M = 1 arm: x [C] -> [1, R] in out_dtype, bias added in fp32
    before the single rounding (src/drinkme/codec/radix_ops.py:351-370)."""
    return gemv_rows(p, x.reshape(1, -1), bias, out_dtype)


def gemv(p: dict, x: torch.Tensor) -> torch.Tensor:
    """The M = 1 arm's fp32 [R] result, no bias (radix_ops.py:373-376)."""
    return gemv_rows(p, x.reshape(1, -1), None, torch.float32).reshape(-1)


def gemv_mc(p: dict, x: torch.Tensor) -> torch.Tensor:
    """x [M, C], 1 <= M <= 8 -> fp32 [M, R] (radix_ops.py:379-398)."""
    return gemv_rows(p, x, None, torch.float32)


class GroupLauncher:
    """dmx_radix_gemv_group over a fixed list of radix tensors that share
    the activation (a layer's q/k/v or gate/up), with the descriptor array
    built once: call(x, biases, out_dtype) for x [..., C] -> one [..., R_i]
    output per tensor, each as gemv_rows would give it (within the same
    float64 bound), in one launch. The descriptors are rebuilt when a
    tensor's runtime dict holds other buffers than at the last call, the
    bias array when the biases are other tensors."""

    def __init__(self, ps):
        ps = list(ps)
        if not ps:
            raise ValueError("radix gemv_group: no tensors")
        if any(_is_twin(p) for p in ps):
            raise ValueError("radix gemv_group: twin dicts launch one GEMV each")
        self.ps = ps
        self.C = int(ps[0]["C"])
        if any(int(p["C"]) != self.C for p in ps):
            raise ValueError(f"radix gemv_group: every tensor needs C = {self.C}")
        self.device = ps[0]["rx_data"].device
        if any(p["rx_data"].device != self.device for p in ps):
            raise ValueError("radix gemv_group: the tensors are on different devices")
        self.R = [int(p["R"]) for p in ps]
        self._held = None
        self._bias_key = None

    def _table(self):
        """The descriptor pointer array, rebuilt when a dict's buffers are no
        longer the ones it was built from."""
        held = [_buffers(p) for p in self.ps]
        if held != self._held:
            descs = [descriptor(p) for p in self.ps]
            self._tarr = (ct.POINTER(_native.RadixTensor) * len(descs))(*[ct.pointer(d) for d in descs])
            self._descs = descs  # the array points into these
            self._held = held
        return self._tarr

    def _bias_array(self, biases, x):
        """(pointer array, dtype code, the biases it points into); kept while
        the same contiguous bias tensors come back at the same addresses."""
        key = tuple(None if b is None else (b.data_ptr(), b.dtype, b.numel()) for b in biases)
        if key == self._bias_key:
            return self._bias_cached
        n = len(self.ps)
        if len(biases) != n:
            raise ValueError("radix gemv_group: one bias (or None) per tensor")
        biases = [None if b is None else b.contiguous() for b in biases]
        dts = {b.dtype for b in biases if b is not None}
        if len(dts) > 1:
            raise ValueError("radix gemv_group: the biases must share a dtype")
        for b, R in zip(biases, self.R):
            if b is not None and (b.numel() != R or b.device != x.device):
                raise ValueError("radix gemv_group: bias must hold R elements on the weight's device")
        bd = _dtype_code(dts.pop(), "bias") if dts else 0
        cached = (ct.c_void_p * n)(*[None if b is None else b.data_ptr() for b in biases]), bd, biases
        # (kept only when no copy was made: the array then points into the
        # callers' own tensors, which the key follows)
        if all(a is None or a[0] == b.data_ptr() for a, b in zip(key, biases)):
            self._bias_key, self._bias_cached = key, cached
        return cached

    def __call__(self, x: torch.Tensor, biases=None, out_dtype=torch.bfloat16) -> list:
        if x.dim() == 0 or x.shape[-1] != self.C:
            raise ValueError(f"radix gemv_group: every tensor needs C = {self.C} and x [..., {self.C}]")
        M = x.numel() // self.C
        if not 1 <= M <= MC_MAX:
            raise ValueError(f"radix gemv_group: M={M} outside 1..{MC_MAX}")
        if x.device != self.device:
            raise ValueError("radix gemv_group: x is not on the weights' device")
        if not x.is_contiguous():
            x = x.contiguous()
        xd = _dtype_code(x.dtype, "activation")
        od = _dtype_code(out_dtype, "output")
        bias_arr, bd = None, 0
        if biases is not None and any(b is not None for b in biases):
            bias_arr, bd, biases = self._bias_array(biases, x)  # (the contiguous biases live through the call)
        tarr = self._table()
        lead = x.shape[:-1]
        outs = [torch.empty((*lead, R), dtype=out_dtype, device=self.device) for R in self.R]
        n = len(outs)
        oarr = (ct.c_void_p * n)(*[o.data_ptr() for o in outs])
        err = _error_buffer()
        st = _native.lib().dmx_radix_gemv_group(tarr, n, x.data_ptr(), xd, M, bias_arr, bd, oarr, od,
                                                 _stream(self.device), err, len(err))
        _native.check(st, err, "dmx_radix_gemv_group")
        return outs


def gemv_group(ps, x: torch.Tensor, biases=None, out_dtype=torch.bfloat16) -> list:
    """Several radix tensors that share the activation (a layer's q/k/v or
    gate/up): x [M, C] or [C] -> one [M, R_i] output per tensor, each as
    gemv_rows would give it (within the same float64 bound), as one launch
    where the kernels allow (dmx_radix_gemv_group; twin dicts launch one
    GEMV each). No drinkme counterpart: drinkme launches one GEMV per
    Linear."""
    ps = list(ps)
    if ps and any(_is_twin(p) for p in ps):  # raw weights: one launch each
        if x.dim() == 1:
            x = x.reshape(1, -1)
        C = int(ps[0]["C"])
        if x.dim() != 2 or x.shape[1] != C or any(int(p["C"]) != C for p in ps):
            raise ValueError(f"radix gemv_group: every tensor needs C = {C} and x [M, {C}]")
        if not 1 <= x.shape[0] <= MC_MAX:
            raise ValueError(f"radix gemv_group: M={x.shape[0]} outside 1..{MC_MAX}")
        bl = list(biases) if biases is not None else [None] * len(ps)
        return [gemv_rows(p, x, b, out_dtype) for p, b in zip(ps, bl)]
    if ps and any(p["rx_data"].device != x.device for p in ps):
        raise ValueError("radix gemv_group: x is not on the weights' device")
    return GroupLauncher(ps)(x.reshape(1, -1) if x.dim() == 1 else x, biases, out_dtype)


def decode_bits(p: dict, num_warps: int | None = None) -> torch.Tensor:
    """Every block once -> the original u16 bit patterns [R, C]
    (radix_ops.py:418-427). `num_warps` is accepted for the signature and
    ignored: the launch shape is the library's."""
    del num_warps
    R, C = int(p["R"]), int(p["C"])
    out = torch.empty((R, C), dtype=torch.uint16, device=p["rx_data"].device)
    err = _native.error_buffer()
    st = _native.lib().dmx_radix_decode(ct.byref(descriptor(p)), out.data_ptr(), _stream(out.device), err, len(err))
    _native.check(st, err, "dmx_radix_decode")
    return out


def decode_weight(p: dict) -> torch.Tensor:
    """The transient bf16 weight [R, C] for F.linear (radix_ops.py:430-432)."""
    return decode_bits(p).view(torch.bfloat16)


def prepare_schedule(data, offsets, C: int, widths, B: int, nblocks: int) -> torch.Tensor:
    """The per-block tier stream lengths, 2 bytes per block, on the device
    (radix_ops.py:341-348). `data` must carry the reach pad."""
    widths = [int(w) for w in widths]
    nb = -(-int(C) // int(B))
    t = _native.RadixTensor()
    t.data = data.data_ptr()
    t.offsets = offsets.data_ptr()
    t.palette = None
    t.schedule = None
    pad = int(_native.lib().dmx_radix_pad_words(int(B), (ct.c_uint32 * 8)(*widths), len(widths)))
    t.payload_words = max(int(data.numel()) - pad, 0)
    t.pad_words = pad
    t.rows, t.cols, t.block_size = int(nblocks) // nb, int(C), int(B)
    t.n_widths = len(widths)
    for i, w in enumerate(widths):
        t.widths[i] = w
    sched = torch.zeros(int(nblocks), dtype=torch.uint16, device=data.device)
    err = _native.error_buffer()
    st = _native.lib().dmx_radix_prepare(ct.byref(t), sched.data_ptr(), _stream(sched.device), err, len(err))
    _native.check(st, err, "dmx_radix_prepare")
    return sched


def read_bytes(p: dict) -> int:
    """Bytes one GEMV call streams: the payload (NW words, not the pad),
    the directory, the tables and the schedule (radix_ops.py:435-441); a
    twin's raw weight."""
    if _is_twin(p):
        return p["weight"].numel() * p["weight"].element_size()
    words = int(p["NW"]) if "NW" in p else p["rx_data"].numel()
    return words * 4 + sum(p[k].numel() * p[k].element_size() for k in ("rx_offsets", "rx_palette", "rx_schedule"))


_POLICIES = {"auto": _native.POLICY_AUTO, "generic": _native.POLICY_GENERIC, "matrix": _native.POLICY_MATRIX}


def set_policy(policy: str) -> str:
    """'auto' (specialised kernels where they apply), 'generic', or
    'matrix' (auto's kernels with gulp's 3- and 4-row verify in quad units
    on the matrix cores, as 8 rows run; no drinkme counterpart); returns the
    previous one. Process-global."""
    code = _POLICIES[policy]
    prev = _native.lib().dmx_radix_set_policy(code)
    return {v: k for k, v in _POLICIES.items()}[prev]
