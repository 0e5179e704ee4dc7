"""GPU: the plain-read probe (dmx_read_probe), the ceiling bench.py times
beside the sweep, reads every byte of its range and nothing else: the XOR of
its workgroups' words equals the XOR of the range's 32-bit words, for
ranges that end inside a 1 KB row, ranges shorter than one row a wave, and
more workgroups than rows; the 64 random words after the range never
enter it."""

import zlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,wgs", [(16, 1), (1008, 3), (1024, 512), (4096 + 16, 7), (1 << 20, 512),
                                        ((1 << 20) + 48, 100), (64 << 20, 512), (3 * 1024 * 1000 + 512, 65535)])
def test_probe_reads_exactly_its_range(cuda, nbytes, wgs):
    import torch

    from drinkme_amd import _native

    rng = np.random.default_rng(zlib.crc32(repr((nbytes, wgs)).encode()))
    words = rng.integers(0, 2**32, size=nbytes // 4 + 64, dtype=np.uint64).astype(np.uint32)
    buf = torch.from_numpy(words.view(np.int32)).to(cuda)
    sink = torch.zeros(wgs, dtype=torch.int32, device=cuda)
    err = _native.error_buffer()
    print(f"case read probe {nbytes} bytes, {wgs} workgroups", flush=True)
    st = _native.lib().dmx_read_probe(buf.data_ptr(), nbytes, sink.data_ptr(), wgs,
                                      torch.cuda.current_stream().cuda_stream, err, len(err))
    _native.check(st, err, "dmx_read_probe")
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    want = np.bitwise_xor.reduce(words[: nbytes // 4])
    assert got == want, f"{nbytes} bytes over {wgs} workgroups: {got:#x} != {want:#x}"
