"""Builds libdmx_radix.so in-tree (drinkme_amd/lib/) for gfx950.

    python -m drinkme_amd.build

The host codec (csrc/codec.cpp) and the pack-file reader and writer
(csrc/pack_io.cpp) are compiled with g++, the kernels (csrc/kernels.hip)
with hipcc for gfx950 only, and all linked into one shared library that
ctypes loads (drinkme_amd/_native.py). Packed-fp32 instructions are
disabled for the device code (-packed-fp32-ops): hipcc otherwise forms
v_pk_*_f32 from scalar float code. The host-only command line tool
lib/dmx_pack (csrc/dmx_pack.cpp) is linked from the same host sources.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libdmx_radix.so")
CLI = os.path.join(LIBDIR, "dmx_pack")
INCLUDE = os.path.join(ROOT, "include")
ARCH = "gfx950"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def _run(cmd, verbose):
    if verbose:
        print("+", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return res


def device_flags() -> list:
    return [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", f"-I{INCLUDE}",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def build(verbose: bool = False) -> str:
    """Compiles and links the library; returns its path."""
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    hipcc = _hipcc()
    host = ["g++", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-Werror", "-pthread", f"-I{INCLUDE}"]
    objs = []
    for src in ("codec", "pack_io", "dmx_pack"):
        obj = os.path.join(OBJ, f"{src}.o")
        _run([*host, "-c", os.path.join(CSRC, f"{src}.cpp"), "-o", obj], verbose)
        objs.append(obj)
    kern_o = os.path.join(OBJ, "kernels.o")
    _run([hipcc, *device_flags(), "-c", os.path.join(CSRC, "kernels.hip"), "-o", kern_o], verbose)
    tmp = LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", objs[0], objs[1], kern_o, "-o", tmp],
         verbose)
    os.replace(tmp, LIB)
    _run(["g++", "-pthread", *objs, "-o", CLI + ".tmp"], verbose)
    os.replace(CLI + ".tmp", CLI)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-q" not in sys.argv))
