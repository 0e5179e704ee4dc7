"""CPU: the C ABI refuses a bad descriptor or bad arguments on the host,
before any device call, with a message naming what is wrong (drinkme's
launchers raise before a launch; its radix_native refuses by name,
src/drinkme/codec/radix_native.cpp:211-236). Each case breaks one rule of
an otherwise valid descriptor; the device pointers are stand-ins that a
refusal never reaches, so the test runs only where no GPU is present."""

import ctypes as ct
import os

import pytest

pytestmark = pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="stand-in device pointers: CPU only")

FAKE = 0x10000  # never dereferenced: every case is refused first


def _tensor(**kw):
    from drinkme_amd import _native

    t = _native.RadixTensor()
    t.data, t.offsets, t.palette, t.schedule = FAKE, FAKE, FAKE, None
    t.rows, t.cols, t.block_size = 8, 2048, 1024
    t.n_widths = 2
    t.widths[0], t.widths[1] = 3, 8
    t.payload_words = 8 * 2 * 400
    t.pad_words = 608
    for k, v in kw.items():
        if k == "widths":
            t.n_widths = len(v)
            for i, w in enumerate(v):
                t.widths[i] = w
        else:
            setattr(t, k, v)
    return t


CASES = [
    ("null descriptor", None, {}, b"null tensor descriptor"),
    ("null payload", {"data": None}, {}, b"null device pointer"),
    ("null directory", {"offsets": None}, {}, b"null device pointer"),
    ("no rows", {"rows": 0}, {}, b"empty tensor"),
    ("no columns", {"cols": 0}, {}, b"empty tensor"),
    ("block not a power of two", {"block_size": 1000}, {}, b"power of two"),
    ("block too large", {"block_size": 8192}, {}, b"power of two"),
    ("block too small", {"block_size": 16}, {}, b"power of two"),
    ("one width", {"widths": (8,)}, {}, b"2..8 widths"),
    ("terminal not 8 bits", {"widths": (3, 7)}, {}, b"2..8 widths"),
    ("a zero width", {"widths": (3, 0, 8)}, {}, b"2..8 widths"),
    ("tiers past the alphabet", {"widths": (8, 8, 8)}, {}, b"exponent alphabet"),
    ("pad short of the reach", {"pad_words": 607}, {}, b"reach pad"),
    ("too many blocks", {"rows": 1 << 30, "cols": 4096}, {}, b"too many blocks"),
    ("null activation", {}, {"x": None}, b"null activation or output"),
    ("null output", {}, {"out": None}, b"null activation or output"),
    ("no rows of x", {}, {"m": 0}, b"m outside 1..8"),
    ("nine rows of x", {}, {"m": 9}, b"m outside 1..8"),
    ("unknown x dtype", {}, {"x_dtype": 5}, b"dtype"),
    ("unknown out dtype", {}, {"out_dtype": 2}, b"dtype"),
]


@pytest.mark.parametrize("name,tkw,akw,msg", CASES, ids=[c[0] for c in CASES])
def test_gemv_refuses_before_any_device_call(name, tkw, akw, msg):
    from drinkme_amd import _native

    L = _native.lib()
    err = _native.error_buffer()
    a = {"x": FAKE, "x_dtype": _native.DMX_BF16, "m": 1, "out": FAKE, "out_dtype": _native.DMX_BF16}
    a.update(akw)
    t = None if tkw is None else _tensor(**tkw)
    st = L.dmx_radix_gemv(None if t is None else ct.byref(t), a["x"], a["x_dtype"], a["m"], None, 0, a["out"],
                          a["out_dtype"], None, err, len(err))
    assert st != 0, f"{name}: accepted"
    assert msg in err.value, f"{name}: {err.value!r}"


def test_group_refusals():
    from drinkme_amd import _native

    L = _native.lib()
    err = _native.error_buffer()
    a, b = _tensor(), _tensor(cols=4096)
    arr = (ct.POINTER(_native.RadixTensor) * 2)(ct.pointer(a), ct.pointer(b))
    outs = (ct.c_void_p * 2)(FAKE, FAKE)
    st = L.dmx_radix_gemv_group(arr, 0, FAKE, _native.DMX_BF16, 1, None, 0, outs, _native.DMX_BF16, None, err,
                                len(err))
    assert st != 0 and b"empty tensor group" in err.value
    st = L.dmx_radix_gemv_group(arr, 2, FAKE, _native.DMX_BF16, 1, None, 0, outs, _native.DMX_BF16, None, err,
                                len(err))
    assert st != 0 and b"share cols" in err.value


PROBE_CASES = [
    ("null data", {"data": None}, b"null data or sink"),
    ("null sink", {"sink": None}, b"null data or sink"),
    ("no bytes", {"bytes": 0}, b"positive multiple of 16"),
    ("ragged bytes", {"bytes": 1000}, b"positive multiple of 16"),
    ("2^31 bytes", {"bytes": 1 << 31}, b"less than 2^31"),
    ("no workgroups", {"sink_words": 0}, b"outside 1..65535"),
    ("too many workgroups", {"sink_words": 65536}, b"outside 1..65535"),
]


@pytest.mark.parametrize("name,kw,msg", PROBE_CASES, ids=[c[0] for c in PROBE_CASES])
def test_read_probe_refuses_before_any_device_call(name, kw, msg):
    from drinkme_amd import _native

    L = _native.lib()
    err = _native.error_buffer()
    a = {"data": FAKE, "bytes": 4096, "sink": FAKE, "sink_words": 512}
    a.update(kw)
    st = L.dmx_read_probe(a["data"], a["bytes"], a["sink"], a["sink_words"], None, err, len(err))
    assert st != 0, f"{name}: accepted"
    assert msg in err.value, f"{name}: {err.value!r}"
