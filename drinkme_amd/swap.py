"""The operator surface over the HIP arms, for drinkme's loader and serving
loop: the resident runtime dict of a packed tensor and the module that
serves it.

Contract kept from drinkme (src/drinkme/codec/swap.py):
  - to_device_radix(pack, device) -> the runtime dict (:80-161): rx_data
    (payload then the reach pad), rx_offsets, rx_palette (padded tier
    tables), rx_schedule (gulp), rx_palette_np and the scalars;
  - RadixCompressedLinear(runtime, bias): M activation rows through one of
    four arms (:302-335, :443-456), the bias added to the fp32 sums before
    the one rounding to x's dtype (:284-300);
  - DRINKME_PREFILL_DENSE_MIN, read once: the row count from which the
    dense arm serves; 0 or less turns it off (:207-224);
  - NarrowLinear / install_narrow (:530-627) and eligible (:850-854): the
    raw bf16 Linears under the codec's row threshold, through gemv_narrow;
  - to_device_twin (:168-196), to_device_raw / RawLinear (:68-77, :459-495)
    and make_module (:900-919).
There is no CPU route: every arm runs on the GPU, and an activation on the
CPU is refused.

Added here, with no drinkme counterpart: SharedInputGroup / install_groups,
which let a layer's q/k/v (and gate/up) modules, still called one by one,
share one grouped launch.
"""

from __future__ import annotations

import os
import warnings
from dataclasses import dataclass

import numpy as np
import torch

from . import radix_ops
from .radix_pack import ARRAYS_RADIX, block_word_bounds, padded_palette_words, validate_radix

FORMAT_VERSION = 1

# ---------------------------------------------------------------- routing --

ENV_DENSE_MIN = "DRINKME_PREFILL_DENSE_MIN"


class RoutePolicy:
    """Which arm serves M activation rows.

        M == 1                         gemv   the fused decode + GEMV
        M >= dense_from (> 0)          dense  decode once, then F.linear
        2 <= M <= MC_MAX otherwise     mc     the same kernels over M rows
        M > MC_MAX, no dense arm       loop   one M = 1 call per row

    dense_from comes from DRINKME_PREFILL_DENSE_MIN the first time it is
    asked for (an unparsable value warns and keeps the default, MC_MAX + 1);
    `override` replaces it, `reset` makes the next call read the environment
    again."""

    default = radix_ops.MC_MAX + 1

    def __init__(self):
        self._dense_from: int | None = None

    @property
    def dense_from(self) -> int:
        if self._dense_from is None:
            text = os.environ.get(ENV_DENSE_MIN, "").strip()
            value = self.default
            if text:
                try:
                    value = int(text)
                except ValueError:
                    warnings.warn(f"{ENV_DENSE_MIN}={text!r} is not an integer; using {self.default}")
            self._dense_from = value
        return self._dense_from

    def override(self, value: int | None) -> None:
        self._dense_from = value

    def reset(self) -> None:
        self._dense_from = None

    def arm(self, m: int) -> str:
        if m == 1:
            return "gemv"
        if 0 < self.dense_from <= m:
            return "dense"
        return "mc" if m <= radix_ops.MC_MAX else "loop"


ROUTES = RoutePolicy()
GEMM_MIN_ROWS = RoutePolicy.default  # src/drinkme/codec/swap.py:251

# ------------------------------------------------------------ runtime dict --


@dataclass(frozen=True)
class _Layout:
    """The device layout of one radix tensor."""
    rows: int
    cols: int
    block: int
    widths: tuple
    blocks: int  # rows x blocks per row
    pad: int     # zero words after the payload: the farthest any block reaches

    @classmethod
    def of(cls, pack: dict) -> "_Layout":
        R, C, B = int(pack["R"]), int(pack["C"]), int(pack["block_size"])
        widths = tuple(int(w) for w in pack["widths"])
        return cls(R, C, B, widths, R * -(-C // B), int(block_word_bounds(B, widths)[1]))


def _upload_u32(arr: np.ndarray, dev: torch.device, extra_zero_words: int = 0) -> torch.Tensor:
    """A u32 host array on the device, followed by extra_zero_words zeros."""
    host = np.ascontiguousarray(arr, dtype=np.uint32).reshape(-1)
    out = torch.empty(host.size + extra_zero_words, dtype=torch.uint32, device=dev)
    out[:host.size].copy_(torch.from_numpy(host))
    if extra_zero_words:
        out[host.size:].zero_()
    return out


def to_device_radix(pack: dict, device="cuda") -> dict:
    """A packed radix tensor (rx_palette, rx_offsets, rx_data + scalars) as
    device buffers, after the descriptor gate (validate_radix):

      rx_data      u32 [NW + pad]  the block streams, then pad zero words
                                   (pad = block_word_bounds(B)[1]: sip 608,
                                   gulp 768): no kernel read of any block
                                   leaves the allocation
      rx_offsets   u32 [NBK + 1]   the word directory
      rx_palette   u32 [...]       each nonterminal tier's entries, padded
                                   with zero bytes to whole words
      rx_schedule  u16 [NBK]       more than two tiers: each block's tier
                                   stream lengths, computed on the device
                                   (dmx_radix_prepare); else empty
    The remaining scalars of the pack dict are kept."""
    validate_radix(pack)
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError("to_device_radix: the radix arms run on the GPU")
    lay = _Layout.of(pack)
    payload_words = int(np.asarray(pack["rx_data"]).size)
    data = _upload_u32(pack["rx_data"], dev, lay.pad)
    offsets = _upload_u32(pack["rx_offsets"], dev)
    tables = _upload_u32(padded_palette_words(pack["rx_palette"], lay.widths), dev)
    schedule = (radix_ops.prepare_schedule(data, offsets, lay.cols, lay.widths, lay.block, lay.blocks)
                if len(lay.widths) > 2 else torch.empty(0, dtype=torch.uint16, device=dev))
    runtime = {k: v for k, v in pack.items() if k not in ARRAYS_RADIX}
    runtime.update(rx_data=data, rx_offsets=offsets, rx_palette=tables, rx_schedule=schedule,
                   rx_palette_np=np.ascontiguousarray(pack["rx_palette"], dtype=np.uint8),
                   NW=payload_words, rx_pad_words=lay.pad, R=lay.rows, C=lay.cols, widths=lay.widths,
                   block_size=lay.block, NBK=lay.blocks, codec="radix", format_version=FORMAT_VERSION, layout=0)
    return runtime


def resident_bytes(p: dict) -> int:
    """Device bytes of a runtime dict: payload + pad, directory, tables,
    schedule."""
    return sum(p[k].numel() * p[k].element_size() for k in ("rx_data", "rx_offsets", "rx_palette", "rx_schedule"))


def to_device_twin(w_bf16, widths=(3, 8), device: str = "cuda") -> dict:
    """A raw bf16 weight [R, C] as a twin dict: the weight resident,
    row-major, codec "twin", with the widths of the compressed tensor it
    stands beside. The GEMV calls of radix_ops run it through that tensor's
    kernel, the decode replaced by a load of the raw weight."""
    w = w_bf16.detach()
    if w.dtype != torch.bfloat16:
        raise TypeError(f"to_device_twin: {w.dtype} is not bf16")
    rows, cols = (int(n) for n in w.shape)
    return {"weight": w.contiguous().to(torch.device(device)), "R": rows, "C": cols,
            "widths": tuple(int(v) for v in widths), "block_size": 1024, "NBK": rows * -(-cols // 1024),
            "codec": "twin", "layout": 0}


def _bits_as_bf16(bits, shape, device) -> torch.Tensor:
    """u16 bit patterns -> a bf16 tensor of `shape` on `device` holding
    exactly those bits (its own copy, never a view of the numpy array)."""
    host = torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)
    return host.reshape(shape).to(torch.device(device), copy=True)


def to_device_raw(pack: dict, device: str = "cuda") -> dict:
    """A tensor stored raw (radix would have expanded it: codec "raw", its
    bf16 bits as raw_bits) as its resident bf16 weight."""
    shape = (int(pack["R"]), int(pack["C"]))
    return dict(weight=_bits_as_bf16(pack["raw_bits"], shape, device), R=shape[0], C=shape[1], codec="raw",
                format_version=FORMAT_VERSION, layout=0)


# ----------------------------------------------------------------- modules --

_KERNEL_DTYPES = (torch.bfloat16, torch.float32)  # activations the kernels take as they are


class RadixCompressedLinear(torch.nn.Module):
    """A radix-coded Linear resident on the GPU (`p` is its runtime dict).

    forward(x [..., C]) -> [..., R] in x's dtype. Each arm accumulates in
    fp32 and adds the bias to the fp32 sums before the only rounding:
      gemv, mc   one launch of radix_ops.gemv_rows for bf16 or fp32 x (bias
                 and rounding in the kernel); other dtypes go through fp32
                 rows and round here
      dense      the weight decoded once (a transient bf16 tensor), then
                 F.linear(x, W, bias): stock's own arithmetic
      loop       one single-row call per activation row"""

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
        self._arms = {"gemv": self._rows_arm, "mc": self._rows_arm, "dense": self._dense_arm,
                      "loop": self._loop_arm}
        self._launch = radix_ops.RowsLauncher(runtime)  # the gemv and mc arms' launch, its descriptor kept
        self._group, self._slot = None, -1  # a SharedInputGroup this module serves in, and its place there

    def _route(self, x) -> str:
        """The arm for x: "cpu" off the GPU, else by its row count (the
        product of its leading dimensions)."""
        return "cpu" if x.device.type == "cpu" else self._route_rows(x.numel() // x.shape[-1])

    @staticmethod
    def _route_rows(m: int) -> str:
        return ROUTES.arm(m)

    def forward(self, x):
        return self._forward(x, self._route(x))

    def _forward(self, x, route: str):
        if route == "cpu":
            raise RuntimeError("RadixCompressedLinear: the radix arms run on the GPU; x is on the CPU")
        if route in ("gemv", "mc") and x.dtype in _KERNEL_DTYPES:  # (output in x's shape, no reshapes)
            if self._group is not None:
                return self._group.rows(self._slot, x)
            return self._launch(x, self.bias, x.dtype)
        rows = x.reshape(-1, self.C)
        y = self._arms[route](rows, x.dtype)
        return y.reshape(*x.shape[:-1], self.R)

    def _round_once(self, y32: torch.Tensor, dtype) -> torch.Tensor:
        """fp32 sums -> + bias in fp32 -> one rounding to dtype."""
        return (y32 if self.bias is None else y32 + self.bias).to(dtype)

    def _rows_arm(self, rows, dtype):
        if dtype in _KERNEL_DTYPES:
            return radix_ops.gemv_rows(self.p, rows, self.bias, dtype)
        return self._round_once(radix_ops.gemv_rows(self.p, rows.float(), None, torch.float32), dtype)

    def _dense_arm(self, rows, dtype):
        weight = radix_ops.decode_weight(self.p)
        return torch.nn.functional.linear(rows if rows.dtype == weight.dtype else rows.to(weight.dtype), weight,
                                          self.bias).to(dtype)

    def _loop_arm(self, rows, dtype):
        sums = torch.empty(rows.shape[0], self.R, device=rows.device, dtype=torch.float32)
        for i in range(rows.shape[0]):
            sums[i:i + 1] = radix_ops.gemv_rows(self.p, rows[i:i + 1].float(), None, torch.float32)
        return self._round_once(sums, dtype)


class RawLinear(torch.nn.Module):
    """A tensor stored raw (to_device_raw): stock's F.linear over the
    resident bf16 weight on every route."""

    def __init__(self, runtime: dict, bias=None):
        super().__init__()
        if runtime.get("codec") != "raw":
            raise ValueError("RawLinear needs a to_device_raw runtime dict")
        self.p = runtime
        self.bias = bias
        self.R, self.C = int(runtime["R"]), int(runtime["C"])
        self.tensor_codec = "raw"
        self.layout = 0

    def forward(self, x):
        return torch.nn.functional.linear(x, self.p["weight"].to(x.device), self.bias)


def make_module(pack: dict, bias=None, device="cuda") -> torch.nn.Module:
    """The served module of one packed tensor, by its codec: radix ->
    RadixCompressedLinear over to_device_radix, raw -> RawLinear."""
    kinds = {"radix": (RadixCompressedLinear, to_device_radix), "raw": (RawLinear, to_device_raw)}
    codec = pack.get("codec")
    if codec not in kinds:
        raise ValueError(f"make_module: codec {codec!r} is not a radix or raw tensor")
    module, resident = kinds[codec]
    return module(resident(pack, device), bias)


# ------------------------------------------------- shared-input groups --


class SharedInputGroup:
    """RadixCompressedLinear modules that read one activation (a decoder
    layer's q/k/v projections, or its gate/up), served by one grouped launch
    (dmx_radix_gemv_group) where drinkme launches one GEMV per module
    (swap.py:443-456). The callers keep calling each module as before.

    The first member called with an activation launches the GEMVs of every
    member and keeps the other members' rows; a member called next with
    that same activation takes its rows from the launch. "That same
    activation" means the same tensor object, at the same address and of the
    same dtype, with torch's version counter unchanged since the launch (no
    in-place write through torch), the same row count, on the same stream
    and under the same graph-capture state.
    The group holds the activation until every member has taken its rows,
    so its memory cannot pass to another tensor meanwhile. Anything else (a
    member called twice, another activation, an in-place write) launches
    again, so each call returns what the module's own launch would (the
    grouped kernels' sums, within the same float64 bound as one GEMV each).
    Not seen: a write into the activation that bypasses torch (a kernel
    given its raw address), or any in-place write to an inference-mode
    tensor (torch keeps no version counter for those); a caller that does
    either between the members' calls calls reset() first."""

    def __init__(self, members):
        members = list(members)
        if len(members) < 2:
            raise ValueError("SharedInputGroup: at least two modules")
        for m in members:
            if not isinstance(m, RadixCompressedLinear):
                raise TypeError(f"SharedInputGroup: {type(m).__name__} is not a RadixCompressedLinear")
            if m._group is not None:
                raise ValueError("SharedInputGroup: a module is already in a group")
        if len({id(m) for m in members}) != len(members):
            raise ValueError("SharedInputGroup: a module appears twice")
        self.launch = radix_ops.GroupLauncher([m.p for m in members])
        self.members = members
        for slot, m in enumerate(members):
            m._group, m._slot = self, slot
        self.reset()

    def reset(self) -> None:
        """Drops the rows held for members not yet called."""
        self._x, self._key, self._outs = None, None, None

    def dissolve(self) -> None:
        """Returns every member to one launch per call."""
        for m in self.members:
            m._group, m._slot = None, -1
        self.reset()

    @staticmethod
    def _match(x, m: int):
        version = None if x.is_inference() else x._version
        return (m, x.data_ptr(), x.dtype, version, radix_ops._stream(x.device), torch.cuda.is_current_stream_capturing())

    def rows(self, slot: int, x: torch.Tensor) -> torch.Tensor:
        """Member `slot`'s rows of activation x [..., C]: [..., R] in x's
        dtype."""
        key = self._match(x, x.numel())
        outs = self._outs
        if outs is None or x is not self._x or key != self._key or outs[slot] is None:
            outs = self.launch(x, [m.bias for m in self.members], x.dtype)
            self._x, self._key, self._outs = x, key, outs
        y, outs[slot] = outs[slot], None
        if all(o is None for o in outs):
            self.reset()
        return y


SIBLINGS = (("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj"))  # children that read one activation


def install_groups(model, sets=SIBLINGS) -> list:
    """Groups, in place, the RadixCompressedLinear children of each module
    of `model` named in one entry of `sets` (at least two present, with one
    column count, device and bias dtype, none grouped yet) into a
    SharedInputGroup; returns the qualified names of each group. Run it
    after the Linears are swapped; nothing else about the modules changes.
    No drinkme counterpart: drinkme launches one GEMV per module."""
    made = []
    for prefix, parent in model.named_modules():
        kids = dict(parent.named_children())
        for names in sets:
            picked = [(n, kids[n]) for n in names
                      if isinstance(kids.get(n), RadixCompressedLinear) and kids[n]._group is None]
            if len(picked) < 2:
                continue
            mods = [m for _, m in picked]
            bias_dtypes = {m.bias.dtype for m in mods if m.bias is not None}
            if (len({m.C for m in mods}) != 1 or len({m.p["rx_data"].device for m in mods}) != 1
                    or len(bias_dtypes) > 1):
                continue
            SharedInputGroup(mods)
            made.append(tuple(f"{prefix}.{n}" if prefix else n for n, _ in picked))
    return made


# ------------------------------------------------------- the raw Linears --


def eligible(child) -> bool:
    """A Linear the codec packs: bf16, columns a multiple of 4, both
    dimensions at least 1024."""
    if not isinstance(child, torch.nn.Linear):
        return False
    rows, cols = child.weight.shape
    return child.weight.dtype == torch.bfloat16 and cols % 4 == 0 and min(rows, cols) >= 1024


class NarrowLinear(torch.nn.Linear):
    """A bf16 Linear the codec leaves raw because it has fewer than 1024
    rows, served on the GPU by radix_ops.gemv_narrow for 1..MC_MAX rows
    (fp32 accumulation, the bias in fp32, one rounding; row m of an M-row
    call equals the one-row call bit for bit) and by F.linear otherwise.
    Its weight and bias are the adopted Linear's own Parameters."""

    BLOCK = 512      # launch knobs of drinkme's kernel (swap.py:577-578),
    NUM_WARPS = 4    # passed through to gemv_narrow, which ignores them
    MAX_ROWS = 1024  # the largest weight this serves: rows ...
    MIN_COLS = 1024  # ... and the shortest: columns

    @classmethod
    def wants(cls, mod) -> bool:
        """A plain torch Linear (not a subclass) the codec does not take,
        with a bf16 GPU weight of at most MAX_ROWS rows and at least
        MIN_COLS columns, a multiple of 4."""
        if type(mod) is not torch.nn.Linear or eligible(mod):
            return False
        w = mod.weight
        rows, cols = w.shape
        fits = rows <= cls.MAX_ROWS and cols >= cls.MIN_COLS and cols % 4 == 0
        return fits and w.dtype == torch.bfloat16 and w.device.type == "cuda"

    @classmethod
    def adopt(cls, lin: torch.nn.Linear) -> "NarrowLinear":
        """A NarrowLinear holding lin's own weight and bias Parameters: no
        copy and no new allocation."""
        mod = cls.__new__(cls)
        torch.nn.Module.__init__(mod)
        mod.in_features, mod.out_features = lin.in_features, lin.out_features
        mod.weight = lin.weight
        mod.register_parameter("bias", lin.bias)
        return mod

    def forward(self, x):
        rows = x.reshape(-1, self.in_features)
        if x.device.type != "cuda" or rows.shape[0] > radix_ops.MC_MAX:
            return torch.nn.functional.linear(x, self.weight, self.bias)
        y = radix_ops.gemv_narrow(self.weight, rows, self.bias, self.BLOCK, self.NUM_WARPS)
        return y.reshape(*x.shape[:-1], self.out_features)


def install_narrow(model, device: str) -> list:
    """Replaces, in place, every child Linear of `model` that
    NarrowLinear.wants by its adopted NarrowLinear; returns [(qualified
    name, (R, C))]. Nothing is replaced off the GPU."""
    if not str(device).startswith("cuda"):
        return []
    found = [(f"{prefix}.{name}" if prefix else name, parent, name, child)
             for prefix, parent in model.named_modules() for name, child in parent.named_children()
             if NarrowLinear.wants(child)]
    for _, parent, name, child in found:
        setattr(parent, name, NarrowLinear.adopt(child))
    return [(qual, tuple(child.weight.shape)) for qual, _, _, child in found]
