"""CPU: the per-tensor pack files (dmx_pack_read / dmx_pack_write and the
dmx_pack command) against NumPy's own reader and writer and against
drinkme's load gates (src/drinkme/codec/pack.py:119-276, :509-520,
:629-644; radix.py:174-238), with the refusal wording drinkme's tests pin
(tests/test_radix_pack.py:647-720, tests/test_radix_bounds.py:392-406).

The files NumPy writes here are written the way PackWriter.add writes them:
np.savez of the codec's arrays plus `scalars`, json.dumps of the scalars in
drinkme's key order.
"""

import hashlib
import json
import os
import subprocess
import zipfile

import numpy as np
import pytest

from drinkme_amd import pack_io, radix_pack as rp, synth
from drinkme_amd.build import CLI
from tests.helpers import finite_bits

SCALARS = {"radix": ("R", "C", "bpw", "codec", "profile", "widths", "block_size"), "raw": ("R", "C", "bpw", "codec")}
ARRAYS = {"radix": ("rx_palette", "rx_offsets", "rx_data"), "raw": ("raw_bits",)}
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.json")


def savez_like_packwriter(path, p, codec=None):
    """PackWriter.add's np.savez (pack.py:509-520)."""
    codec = codec or p["codec"]
    np.savez(path, **{k: p[k] for k in ARRAYS[codec]},
             scalars=np.array([json.dumps({k: p[k] for k in SCALARS[codec] if k in p})]))
    return str(path) if str(path).endswith(".npz") else str(path) + ".npz"


def _probe(profile="sip", R=64, C=2048, seed=3):
    return rp.pack_array_radix(finite_bits(np.random.default_rng(seed), (R, C)), profile)


@pytest.mark.parametrize("profile", ["sip", "gulp", "balanced"])
def test_read_gives_back_what_numpy_wrote(tmp_path, profile):
    p = _probe(profile)
    fn = savez_like_packwriter(tmp_path / "t", p)
    q = pack_io.read_tensor(fn, "a")
    for k in ARRAYS["radix"]:
        assert q[k].dtype == p[k].dtype and np.array_equal(q[k], p[k]), k
    for k in SCALARS["radix"]:
        assert q[k] == p[k], k
    assert q["format_version"] == 1


def test_raw_tensor_reads_back(tmp_path):
    U = finite_bits(np.random.default_rng(4), (16, 1024))
    fn = savez_like_packwriter(tmp_path / "r", rp.raw_dict(U))
    q = pack_io.read_tensor(fn, "a")
    assert q["codec"] == "raw" and q["bpw"] == 16.0 and np.array_equal(q["raw_bits"], U)


@pytest.mark.parametrize("codec", ["radix", "raw"])
def test_written_file_is_what_numpy_reads_and_what_json_dumps_writes(tmp_path, codec):
    p = _probe("gulp") if codec == "radix" else rp.raw_dict(finite_bits(np.random.default_rng(5), (8, 1030)))
    fn = str(tmp_path / "w.npz")
    pack_io.write_tensor(fn, p)
    with np.load(fn) as z:  # np.load checks every member's CRC
        assert sorted(z.files) == sorted(ARRAYS[codec] + ("scalars",))
        for k in ARRAYS[codec]:
            assert z[k].dtype == np.asarray(p[k]).dtype and np.array_equal(z[k], p[k]), k
        assert str(z["scalars"][0]) == json.dumps({k: p[k] for k in SCALARS[codec]})
    with zipfile.ZipFile(fn) as zf:
        assert zf.testzip() is None
        assert all(i.compress_type == zipfile.ZIP_STORED for i in zf.infolist())
    q = pack_io.read_tensor(fn)
    for k in ARRAYS[codec]:
        assert np.array_equal(q[k], p[k])


def test_zip64_local_headers_are_read(tmp_path):
    """NumPy and zipfile may write ZIP64 extras into local headers."""
    p = _probe()
    fn = str(tmp_path / "z64.npz")
    with zipfile.ZipFile(fn, "w") as zf:
        for k in ARRAYS["radix"]:
            with zf.open(k + ".npy", "w", force_zip64=True) as f:
                np.lib.format.write_array(f, np.asarray(p[k]))
        with zf.open("scalars.npy", "w", force_zip64=True) as f:
            np.lib.format.write_array(f, np.array([json.dumps({k: p[k] for k in SCALARS["radix"]})]))
    q = pack_io.read_tensor(fn)
    assert np.array_equal(q["rx_data"], p["rx_data"])


@pytest.mark.parametrize("field,value,why", [
    ("widths", [2, 2, 2, 2, 8], "tiers"),
    ("widths", [5, 8], "nonterminal"),
    ("block_size", 512, "block_size"),
    ("R", 63, "invalid radix block offsets"),
    ("C", 2049, "invalid radix block offsets"),
])
def test_descriptors_the_served_kernels_cannot_take_are_refused_by_name(tmp_path, field, value, why):
    p = dict(_probe(), **{field: value})
    fn = savez_like_packwriter(tmp_path / "bad", p)
    with pytest.raises(ValueError, match=f"pack tensor a \\(radix\\).*{why}"):
        pack_io.read_tensor(fn, "a")


def test_widths_profile_and_codec_refusals(tmp_path):
    p = _probe()
    for bad, msg in (({"widths": [3]}, r"widths \[3\] is not a list of 2\+ ints"),
                     ({"widths": [3, 9]}, "the terminal tier is the 8-bit bf16 exponent"),
                     ({"profile": "fast"}, r"profile 'fast' is not one this drinkme packs or serves \(sip \| gulp\)"),
                     ({"codec": "zstd"}, r"pack tensor a declares codec 'zstd', which this build does not implement "
                                         r"\(knows 'radix' and 'raw'\) — refusing to load\.")):
        fn = savez_like_packwriter(tmp_path / "b", dict(p, **bad), codec="radix")
        with pytest.raises(ValueError, match=msg):
            pack_io.read_tensor(fn, "a")
    fn = str(tmp_path / "nocodec.npz")
    np.savez(fn, scalars=np.array([json.dumps({"R": 1, "C": 1})]))
    with pytest.raises(ValueError, match=r"pack tensor a names no codec \('radix' \| 'raw'\) — not a pack format 1"):
        pack_io.read_tensor(fn, "a")


def test_raw_tensor_shape_and_dtype_are_checked(tmp_path):
    U = finite_bits(np.random.default_rng(4), (16, 1024))
    fn = savez_like_packwriter(tmp_path / "s", dict(rp.raw_dict(U), raw_bits=U[:8]))
    with pytest.raises(ValueError, match=r"pack tensor a \(raw\): raw_bits is \(8, 1024\), not \[R, C\] = \(16, 1024\)"):
        pack_io.read_tensor(fn, "a")
    # (a uint32 array the size of the plane: past the allocation cap, to the dtype gate)
    fn = savez_like_packwriter(tmp_path / "d", dict(rp.raw_dict(U), raw_bits=U[:, :512].astype(np.uint32)))
    with pytest.raises(ValueError, match="raw_bits dtype uint32, not uint16"):
        pack_io.read_tensor(fn, "a")
    fn = savez_like_packwriter(tmp_path / "big", dict(rp.raw_dict(U), raw_bits=U.astype(np.uint32)))
    with pytest.raises(ValueError, match=r"raw_bits.npy is 65,664 bytes, more than the 2 x R x C = 32,768 bytes of "
                                         r"bf16 bits it declares"):
        pack_io.read_tensor(fn, "a")


def test_allocation_is_capped_off_the_zip_directory(tmp_path):
    p = _probe()
    fn = savez_like_packwriter(tmp_path / "cap", dict(p, R=1, C=1024))
    with pytest.raises(ValueError, match=r"pack tensor a \(radix\): rx_data.npy is .* bytes, more than the "
                                         r"2 x R x C = 2,048 the tensor's bf16 plane takes — refusing to allocate it"):
        pack_io.read_tensor(fn, "a")
    fn = savez_like_packwriter(tmp_path / "noraw", dict(p, codec="raw"), codec="radix")
    with pytest.raises(ValueError, match=r"declares R x C = 64 x 2048 but the npz holds no raw_bits.npy "
                                         r"\(members: \['rx_data.npy', 'rx_offsets.npy', 'rx_palette.npy', "
                                         r"'scalars.npy'\]\)"):
        pack_io.read_tensor(fn, "a")
    fn = savez_like_packwriter(tmp_path / "huge", dict(p, R=2 ** 32, C=4))
    with pytest.raises(ValueError, match=r"pack tensor a \(radix\): R x C = 4,294,967,296 x 4 is 17,179,869,184 "
                                         r"weights, more than the 8,589,934,592 this loader will allocate for"):
        pack_io.read_tensor(fn, "a")
    fn = savez_like_packwriter(tmp_path / "zero", dict(p, R=0))
    with pytest.raises(ValueError, match=r"R, C must be positive ints, got 0, 2048"):
        pack_io.read_tensor(fn, "a")


def test_directories_that_contradict_the_codec_are_refused(tmp_path):
    """drinkme's tests/test_radix_bounds.py:392-406: a block pointing into
    the previous one, and a block longer than any block can be."""
    p = _probe(R=4, C=1024)
    off = p["rx_offsets"].copy()
    off[1] = off[0] + 100
    fn = savez_like_packwriter(tmp_path / "into", dict(p, rx_offsets=off))
    with pytest.raises(ValueError, match="block 0 holds 100 word.*fewer than the 352 its literal plane and first tier "
                                         "take for 1024 weights"):
        pack_io.read_tensor(fn, "a")
    grow = 609 - int(p["rx_offsets"][2] - p["rx_offsets"][1])
    data = np.concatenate([p["rx_data"][:p["rx_offsets"][2]], np.zeros(grow, np.uint32), p["rx_data"][p["rx_offsets"][2]:]])
    off = p["rx_offsets"].copy()
    off[2:] += grow
    fn = savez_like_packwriter(tmp_path / "over", dict(p, rx_offsets=off, rx_data=data))
    with pytest.raises(ValueError, match="block 1 holds 609 words, more than the 608 any block of 1024 weights"):
        pack_io.read_tensor(fn, "a")


def test_files_that_are_not_stored_npz_are_refused(tmp_path):
    p = _probe()
    fn = str(tmp_path / "c.npz")
    np.savez_compressed(fn, **{k: p[k] for k in ARRAYS["radix"]},
                        scalars=np.array([json.dumps({k: p[k] for k in SCALARS["radix"]})]))
    with pytest.raises(ValueError, match="compressed ZIP member"):
        pack_io.read_tensor(fn, "a")
    junk = tmp_path / "junk.npz"
    junk.write_bytes(b"not a zip at all" * 10)
    with pytest.raises(ValueError, match="not a ZIP archive"):
        pack_io.read_tensor(str(junk), "a")
    with pytest.raises(ValueError, match="No such file"):
        pack_io.read_tensor(str(tmp_path / "missing.npz"), "a")


def _cli(*args):
    return subprocess.run([CLI, *map(str, args)], capture_output=True, text=True, timeout=300)


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.mark.parametrize("profile", ["sip", "gulp", "balanced"])
def test_cli_encodes_drinkmes_golden_bytes(tmp_path, profile):
    """The command packs the golden case with drinkme's encoder's bytes
    (the SHA-256 digests tests/golden/make_golden.py recorded from
    radix_native.cpp) and writes them as a pack tensor file."""
    case = json.load(open(GOLDEN))["cases"]["gate_1024x4096_normal"]
    bits = synth.weight("qwen3-8b", 0, "gate", 1024, 4096)
    assert _sha(bits) == case["source_sha256"]
    src, out = tmp_path / "src.npy", tmp_path / "out.npz"
    np.save(src, bits)
    r = _cli("encode", "--profile", profile, "--threads", "3", src, out)
    assert r.returncode == 0, r.stderr
    g = case["profiles"][profile]
    with np.load(out) as z:
        assert _sha(z["rx_palette"]) == g["palette_sha256"]
        assert _sha(z["rx_offsets"]) == g["offsets_sha256"]
        assert _sha(z["rx_data"]) == g["data_sha256"]
        sc = json.loads(str(z["scalars"][0]))
    assert sc["profile"] == profile and sc["widths"] == list(rp.widths_of(profile)) and sc["codec"] == "radix"
    stored = len(g["palette"]) + 4 * (1024 * 4 + 1) + 4 * g["words"]
    assert sc["bpw"] == 8.0 * stored / (1024 * 4096)
    # and the Python packer writes the same tensor
    p = rp.pack_array_radix(bits, profile)
    assert sc == {k: p[k] for k in SCALARS["radix"]}
    r = _cli("verify", out, src)
    assert r.returncode == 0 and "equal to the source" in r.stdout, r.stderr
    back = tmp_path / "back.npy"
    assert _cli("decode", out, back).returncode == 0
    assert np.array_equal(np.load(back), bits)
    info = json.loads(_cli("info", out).stdout)
    assert info["R"] == 1024 and info["data_words"] == g["words"]


def test_cli_falls_back_to_raw_where_radix_would_expand(tmp_path):
    """Uniform random bit patterns: radix would not compress them (most
    exponents escape every tier), so the tensor is stored raw, as
    pack_array_radix's caller stores it."""
    a = np.random.default_rng(8).integers(0, 1 << 16, (64, 1030), dtype=np.uint16)
    assert rp.pack_array_radix(a, "sip") is None
    src, out = tmp_path / "src.npy", tmp_path / "out.npz"
    np.save(src, a)
    assert _cli("encode", src, out).returncode == 0
    q = pack_io.read_tensor(str(out))
    assert q["codec"] == "raw" and q["bpw"] == 16.0 and np.array_equal(q["raw_bits"], a)


def test_cli_refuses_by_name(tmp_path):
    src = tmp_path / "f.npy"
    np.save(src, np.zeros((4, 4), np.float32))
    r = _cli("encode", src, tmp_path / "o.npz")
    assert r.returncode == 1 and "uint16" in r.stderr
    r = _cli("encode", "--profile", "tiny", src, tmp_path / "o.npz")
    assert r.returncode == 1 and "unknown profile 'tiny'" in r.stderr
    p = dict(_probe(), block_size=512)
    fn = savez_like_packwriter(tmp_path / "bad", p)
    r = _cli("verify", fn)
    assert r.returncode == 1 and "the served kernels walk 1024-weight blocks only" in r.stderr
