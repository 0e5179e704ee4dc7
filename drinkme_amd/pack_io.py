"""drinkme's per-tensor pack files over libdmx_radix.so, without np.load or
np.savez: one tensor of a pack is one .npz (stored .npy members plus a
`scalars` JSON blob).

  read_tensor(path, name)   the dict pack._read_tensor returns
                            (src/drinkme/codec/pack.py:629-644): the codec's
                            arrays and scalars, format_version 1, after
                            drinkme's load gates; refusals raise ValueError
                            with drinkme's message
  write_tensor(path, pack)  the file PackWriter.add writes (pack.py:509-520)

The command-line form of the same step is lib/dmx_pack (encode, decode,
info, verify), built beside the library.

    python -m drinkme_amd.pack_io [--rows R] [--cols C] [--profile P]

times it against drinkme's NumPy route on one synthetic tensor file (one
JSON line).
"""

from __future__ import annotations

import ctypes as ct

import numpy as np

from . import _native
from .radix_pack import RADIX, RAW

FORMAT_VERSION = 1


def _read(path: str, name: str, info, *bufs):
    err = _native.error_buffer()
    ptrs = [None if b is None else b.ctypes.data for b in bufs]
    st = _native.lib().dmx_pack_read(path.encode(), name.encode(), ct.byref(info), *ptrs, err, len(err))
    if st:
        raise ValueError(err.value.decode(errors="replace"))


def read_tensor(path: str, name: str = "a") -> dict:
    """One tensor file -> its runtime-ready dict (arrays + scalars +
    format_version), through the codec, size and descriptor gates."""
    info = _native.PackInfo()
    _read(str(path), name, info, None, None, None, None)
    R, C = int(info.rows), int(info.cols)
    p = {"R": R, "C": C, "bpw": float(info.bpw)}
    if info.codec == _native.DMX_CODEC_RAW:
        bits = np.empty((R, C), dtype=np.uint16)
        _read(str(path), name, info, None, None, None, bits)
        p.update(raw_bits=bits, codec=RAW)
    else:
        pal = np.empty(int(info.palette_len), dtype=np.uint8)
        off = np.empty(int(info.offsets_len), dtype=np.uint32)
        data = np.empty(int(info.data_len), dtype=np.uint32)
        _read(str(path), name, info, pal, off, data, None)
        p.update(rx_palette=pal, rx_offsets=off, rx_data=data, codec=RADIX, profile=info.profile.decode(),
                 widths=[int(info.widths[k]) for k in range(info.n_widths)], block_size=int(info.block_size))
    p["format_version"] = FORMAT_VERSION
    return p


def write_tensor(path: str, pack: dict) -> None:
    """A radix or raw tensor dict -> its .npz, as PackWriter.add writes it."""
    info = _native.PackInfo()
    info.rows, info.cols = int(pack["R"]), int(pack["C"])
    info.bpw = float(pack["bpw"])
    bufs = [None, None, None, None]
    if pack.get("codec") == RADIX:
        widths = [int(w) for w in pack["widths"]]
        if not 2 <= len(widths) <= 8:
            raise ValueError("write_tensor: radix needs 2..8 widths")
        info.codec = _native.DMX_CODEC_RADIX
        info.block_size = int(pack["block_size"])
        info.n_widths = len(widths)
        for k, w in enumerate(widths):
            info.widths[k] = w
        info.profile = str(pack["profile"]).encode()
        bufs[:3] = [np.ascontiguousarray(pack["rx_palette"], dtype=np.uint8),
                    np.ascontiguousarray(pack["rx_offsets"], dtype=np.uint32),
                    np.ascontiguousarray(pack["rx_data"], dtype=np.uint32)]
        info.palette_len, info.offsets_len, info.data_len = (b.size for b in bufs[:3])
    elif pack.get("codec") == RAW:
        info.codec = _native.DMX_CODEC_RAW
        bits = np.ascontiguousarray(pack["raw_bits"], dtype=np.uint16)
        if bits.shape != (info.rows, info.cols):
            raise ValueError(f"write_tensor: raw_bits is {bits.shape}, not [R, C] = ({info.rows}, {info.cols})")
        bufs[3] = bits
    else:
        raise ValueError("write_tensor: a pack dict must be a radix or raw tensor")
    err = _native.error_buffer()
    st = _native.lib().dmx_pack_write(str(path).encode(), ct.byref(info),
                                      *[None if b is None else b.ctypes.data for b in bufs], err, len(err))
    if st:
        raise ValueError(err.value.decode(errors="replace"))


def _bench(argv=None) -> int:
    """NumPy's route (np.load of the arrays, then the descriptor gate in
    NumPy, as pack._read_tensor runs them) against read_tensor, and the
    Python packer against the dmx_pack command, on one tensor file in the
    page cache."""
    import argparse
    import json
    import os
    import subprocess
    import tempfile
    import time

    from . import radix_pack, synth
    from .build import CLI

    ap = argparse.ArgumentParser()
    ap.add_argument("--rows", type=int, default=12288)
    ap.add_argument("--cols", type=int, default=4096)
    ap.add_argument("--profile", default="sip", choices=["sip", "gulp", "balanced"])
    ap.add_argument("--reps", type=int, default=5)
    a = ap.parse_args(argv)
    bits = synth.weight("qwen3-8b", 0, "gate", a.rows, a.cols)

    def best(fn):
        t = []
        for _ in range(a.reps):
            t0 = time.perf_counter()
            fn()
            t.append(time.perf_counter() - t0)
        return min(t)

    with tempfile.TemporaryDirectory() as d:
        src, npz = os.path.join(d, "src.npy"), os.path.join(d, "t.npz")
        np.save(src, bits)
        enc_py = best(lambda: radix_pack.pack_array_radix(bits, a.profile))
        enc_cli = best(lambda: subprocess.run([CLI, "encode", "--profile", a.profile, src, npz], check=True,
                                              capture_output=True))
        size = os.path.getsize(npz)

        def numpy_route():
            with np.load(npz) as z:
                sc = json.loads(str(z["scalars"][0]))
                p = {k: np.asarray(z[k]) for k in ("rx_palette", "rx_offsets", "rx_data")}
            p.update(sc)
            radix_pack.validate_radix(p)

        t_np = best(numpy_route)
        t_dmx = best(lambda: read_tensor(npz))
    print(json.dumps({"what": "one pack tensor file", "shape": [a.rows, a.cols], "profile": a.profile,
                      "file_bytes": size, "read_numpy_s": t_np, "read_dmx_s": t_dmx,
                      "read_numpy_GBps": size / t_np / 1e9, "read_dmx_GBps": size / t_dmx / 1e9,
                      "encode_python_s": enc_py, "encode_cli_s": enc_cli,
                      "encode_note": "both run dmx_radix_native plan + encode + the CPU round trip; the command "
                                     "also reads the .npy and writes the .npz",
                      "host_threads": _native.lib().dmx_set_host_threads(0)}))
    return 0


if __name__ == "__main__":
    raise SystemExit(_bench())
