"""ctypes binding of libdmx_radix.so (include/dmx_radix.h).

The library is built in-tree by `python -m drinkme_amd.build` (or
__graft_entry__.build()). There is no fallback: a missing library raises
here, at first use, with the path it looked for.
"""

from __future__ import annotations

import ctypes as ct
import os

from .build import LIB

DMX_BF16 = 0
DMX_F32 = 1
POLICY_AUTO = 0
POLICY_GENERIC = 1
POLICY_MATRIX = 2  # AUTO, with gulp's 3- and 4-row verify on the matrix cores


class RadixTensor(ct.Structure):
    """dmx_radix_tensor."""
    _fields_ = [
        ("data", ct.c_void_p),
        ("offsets", ct.c_void_p),
        ("palette", ct.c_void_p),
        ("schedule", ct.c_void_p),
        ("payload_words", ct.c_uint64),
        ("pad_words", ct.c_uint64),
        ("rows", ct.c_uint32),
        ("cols", ct.c_uint32),
        ("block_size", ct.c_uint32),
        ("n_widths", ct.c_uint32),
        ("widths", ct.c_uint32 * 8),
    ]


class PackInfo(ct.Structure):
    """dmx_pack_info."""
    _fields_ = [
        ("codec", ct.c_uint32),
        ("block_size", ct.c_uint32),
        ("rows", ct.c_uint64),
        ("cols", ct.c_uint64),
        ("n_widths", ct.c_uint32),
        ("widths", ct.c_uint32 * 8),
        ("profile", ct.c_char * 16),
        ("bpw", ct.c_double),
        ("palette_len", ct.c_uint64),
        ("offsets_len", ct.c_uint64),
        ("data_len", ct.c_uint64),
    ]


DMX_CODEC_RADIX = 0
DMX_CODEC_RAW = 1

# every symbol include/dmx_radix.h declares, with its ctypes signature
_P, _U64, _U32, _I, _SZ = ct.c_void_p, ct.c_uint64, ct.c_uint32, ct.c_int, ct.c_size_t
_TP = ct.POINTER(RadixTensor)
SIGNATURES = {
    "dmx_abi_version": (_I, []),
    "dmx_radix_pad_words": (_U64, [_U32, _P, _U32]),
    "dmx_radix_native": (_I, [_U32, _P, _U64, _U64, _U64, _U64, _U32, _U32, _P, _U32, _P, _P, _P, _U64, _U64, _U64,
                              _P, _P, _U64]),
    "dmx_set_host_threads": (_I, [_I]),
    "dmx_radix_decode": (_I, [_TP, _P, _P, _P, _SZ]),
    "dmx_radix_prepare": (_I, [_TP, _P, _P, _P, _SZ]),
    "dmx_radix_gemv": (_I, [_TP, _P, _I, _U32, _P, _I, _P, _I, _P, _P, _SZ]),
    "dmx_radix_gemv_group": (_I, [_P, _U32, _P, _I, _U32, _P, _I, _P, _I, _P, _P, _SZ]),
    "dmx_gemv_narrow": (_I, [_P, _U32, _U32, _P, _I, _U32, _P, _I, _P, _I, _P, _P, _SZ]),
    "dmx_radix_gemv_twin": (_I, [_P, _U32, _U32, _U32, _U32, _P, _P, _I, _U32, _P, _I, _P, _I, _P, _P, _SZ]),
    "dmx_pack_read": (_I, [ct.c_char_p, ct.c_char_p, _P, _P, _P, _P, _P, _P, _SZ]),
    "dmx_pack_write": (_I, [ct.c_char_p, _P, _P, _P, _P, _P, _P, _SZ]),
    "dmx_radix_set_policy": (_I, [_I]),
    "dmx_read_probe": (_I, [_P, _U64, _P, _U32, _P, _P, _SZ]),
    "dmx_synth_bf16": (_I, [_U64, _U64, _U64, ct.c_double, _U32, _P, _P, _SZ]),
}

_lib = None


def lib():
    """The loaded library (raises when it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise ImportError(f"libdmx_radix.so is not built ({LIB}); run `python -m drinkme_amd.build`")
        L = ct.CDLL(LIB)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        if L.dmx_abi_version() != 1:
            raise ImportError(f"{LIB}: ABI version {L.dmx_abi_version()}, expected 1")
        _lib = L
    return _lib


def error_buffer():
    return ct.create_string_buffer(512)


def check(status: int, err, what: str) -> None:
    if status:
        raise RuntimeError(f"{what}: {err.value.decode(errors='replace')}")
