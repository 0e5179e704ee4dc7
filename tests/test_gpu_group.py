"""GPU parity: the grouped launch (dmx_radix_gemv_group) — several tensors
sharing one activation — against the oracle, through the C ABI.

Each output must meet the same bars as a single dmx_radix_gemv: within the
float64 bound of the oracle's dot over the source bits, the fused bias
epilogue exact. The groups mix exponent distributions so the tensors'
palettes differ, and their row counts put tensor boundaries inside
workgroup tiles (a workgroup then holds two tensors' tables)."""

import zlib

import numpy as np
import pytest

from oracle import radix_oracle as O
from tests.helpers import bf16_tensor, escape_heavy_bits, finite_bits, oracle_dict

pytestmark = pytest.mark.gpu


def _bits(rng, shape, kind):
    if kind == "tight":
        return finite_bits(rng, shape, spread=False)
    if kind == "spread":
        return finite_bits(rng, shape, spread=True)
    return escape_heavy_bits(rng, shape, 0.05)


def _check(y, xf, bits, what):
    ref, bound = O.gemv_f64(bits, xf)
    err = np.abs(np.asarray(y, np.float64).reshape(ref.shape) - ref) / bound
    assert np.all(err <= 1.0), f"{what}: err/bound {err.max():.3f}"


@pytest.mark.parametrize("rows", [(4096, 1024, 1024), (12288, 12288), (1000, 37, 2000), (5, 7), (300, 301, 302, 303),
                                  (2048,)])
@pytest.mark.parametrize("C,M", [(4096, 1), (2048, 1), (4096, 4), (2048, 3), (1024, 8)])
def test_group_matches_the_oracle(cuda, rows, C, M):
    import torch

    from drinkme_amd import radix_ops, swap

    rng = np.random.default_rng(zlib.crc32(repr((rows, C, M)).encode()))
    kinds = ("tight", "spread", "escapes", "tight")
    bits = [_bits(rng, (r, C), kinds[i % 4]) for i, r in enumerate(rows)]
    rts = [swap.to_device_radix(oracle_dict(b, "sip"), cuda) for b in bits]
    assert len({tuple(rt["rx_palette_np"]) for rt in rts}) > 1 or len(rts) == 1
    xb = O.f32_to_bf16_bits(rng.standard_normal((M, C)).astype(np.float32))
    x = bf16_tensor(xb, cuda)
    xf = O.bf16_bits_to_f32(xb)
    print(f"case group rows={rows} C={C} M={M}", flush=True)
    ys = radix_ops.gemv_group(rts, x, None, torch.float32)
    for i, (y, b) in enumerate(zip(ys, bits)):
        _check(y.cpu().numpy(), xf, b, f"group {rows} tensor {i}")
    # biases (one missing), bf16 out: the epilogue rounds the fp32 sum once
    biases = [None if i == 1 else bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal(r).astype(np.float32)), cuda)
              for i, r in enumerate(rows)]
    fused = radix_ops.gemv_group(rts, x, biases, torch.bfloat16)
    for i, (f, y) in enumerate(zip(fused, ys)):
        want = y if biases[i] is None else y + biases[i].float()
        assert torch.equal(f, want.to(torch.bfloat16)), f"group {rows} tensor {i}: fused epilogue"
    # twice more: deterministic
    again = radix_ops.gemv_group(rts, x, None, torch.float32)
    assert all(torch.equal(a, b) for a, b in zip(again, ys))


@pytest.mark.parametrize("rows,C,M", [((4096, 1024, 1024), 4096, 1), ((4096, 1024, 1024), 4096, 2),
                                      ((4096, 1024, 1024), 4096, 4),
                                      ((8192, 1024, 1024), 5120, 1), ((12288, 12288), 4096, 1),
                                      ((640, 128, 128), 1024, 8), ((1000, 37, 2000), 2048, 1)])
def test_gulp_group_matches_the_oracle(cuda, rows, C, M):
    """gulp groups: the kernel keeps one tensor per workgroup, so q/k/v-like
    groups run as one launch with a tile height that divides every tensor
    boundary (8 rows for 4096/1024/1024: 768 tiles, so 8-wave workgroups,
    three per CU, at M = 1, 2 and 4); a group with no such height
    (1000/37/2000) runs tensor by tensor. Same bars as sip."""
    import torch

    from drinkme_amd import radix_ops, swap

    rng = np.random.default_rng(zlib.crc32(repr(("gulp", rows, C, M)).encode()))
    kinds = ("tight", "spread", "escapes")
    bits = [_bits(rng, (r, C), kinds[i % 3]) for i, r in enumerate(rows)]
    rts = [swap.to_device_radix(oracle_dict(b, "gulp"), cuda) for b in bits]
    xb = O.f32_to_bf16_bits(rng.standard_normal((M, C)).astype(np.float32))
    x = bf16_tensor(xb, cuda)
    xf = O.bf16_bits_to_f32(xb)
    print(f"case gulp group rows={rows} C={C} M={M}", flush=True)
    ys = radix_ops.gemv_group(rts, x, None, torch.float32)
    for i, (y, b) in enumerate(zip(ys, bits)):
        _check(y.cpu().numpy(), xf, b, f"gulp group {rows} tensor {i}")
    biases = [bf16_tensor(O.f32_to_bf16_bits(rng.standard_normal(r).astype(np.float32)), cuda) for r in rows]
    fused = radix_ops.gemv_group(rts, x, biases, torch.bfloat16)
    for i, (f, y) in enumerate(zip(fused, ys)):
        assert torch.equal(f, (y + biases[i].float()).to(torch.bfloat16)), f"gulp group {rows} tensor {i}: epilogue"
    again = radix_ops.gemv_group(rts, x, None, torch.float32)
    assert all(torch.equal(a, b) for a, b in zip(again, ys))


def test_group_fallbacks_match_the_oracle(cuda):
    """Groups the one-launch kernel does not take run tensor by tensor:
    more than four tensors, a tensor shorter than the row tile, a gulp
    member, M = 3, fp32 activations."""
    import torch

    from drinkme_amd import radix_ops, swap

    rng = np.random.default_rng(77)
    C = 1024
    cases = {
        "six tensors": [(r, "sip") for r in (64, 65, 66, 67, 68, 69)],
        "short tensor": [(8000, "sip"), (3, "sip")],
        "gulp member": [(512, "sip"), (512, "gulp")],
    }
    for name, spec in cases.items():
        bits = [finite_bits(rng, (r, C), spread=True) for r, _ in spec]
        rts = [swap.to_device_radix(oracle_dict(b, prof), cuda) for b, (_, prof) in zip(bits, spec)]
        for M, xdt in ((1, torch.bfloat16), (3, torch.bfloat16), (1, torch.float32)):
            xb = O.f32_to_bf16_bits(rng.standard_normal((M, C)).astype(np.float32))
            x = bf16_tensor(xb, cuda).to(xdt)
            print(f"case group fallback {name} M={M} {xdt}", flush=True)
            ys = radix_ops.gemv_group(rts, x, None, torch.float32)
            for i, (y, b) in enumerate(zip(ys, bits)):
                _check(y.cpu().numpy(), O.bf16_bits_to_f32(xb), b, f"{name} M={M} tensor {i}")


def test_group_refuses_unequal_cols_and_launches_nothing(cuda):
    import torch

    from drinkme_amd import _native, radix_ops, swap

    rng = np.random.default_rng(5)
    a = swap.to_device_radix(oracle_dict(finite_bits(rng, (8, 1024)), "sip"), cuda)
    b = swap.to_device_radix(oracle_dict(finite_bits(rng, (8, 2048)), "sip"), cuda)
    x = torch.zeros(1024, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(ValueError, match="C = 1024"):
        radix_ops.gemv_group([a, b], x)
    # the C ABI itself refuses too
    import ctypes as ct

    descs = [radix_ops.descriptor(a), radix_ops.descriptor(b)]
    tarr = (ct.POINTER(_native.RadixTensor) * 2)(*[ct.pointer(d) for d in descs])
    outs = [torch.empty(8, dtype=torch.float32, device=cuda) for _ in range(2)]
    oarr = (ct.c_void_p * 2)(*[o.data_ptr() for o in outs])
    err = _native.error_buffer()
    st = _native.lib().dmx_radix_gemv_group(tarr, 2, x.data_ptr(), 0, 1, None, 0, oarr, 1, None, err, len(err))
    assert st != 0 and b"cols" in err.value
