"""Host-side checks of the operator surface (drinkme_amd/swap.py) that need
no GPU: the route policy of src/drinkme/codec/swap.py:207-224, :302-335
(DRINKME_PREFILL_DENSE_MIN read once, an unparsable value warned about and
replaced by the default, 0 or less turning the dense arm off) and the raw
tensor's module (:68-77, :459-495)."""

import numpy as np
import pytest
import torch

from drinkme_amd import radix_ops, swap


def _policy(monkeypatch, value):
    if value is None:
        monkeypatch.delenv(swap.ENV_DENSE_MIN, raising=False)
    else:
        monkeypatch.setenv(swap.ENV_DENSE_MIN, value)
    return swap.RoutePolicy()


def test_default_routes(monkeypatch):
    pol = _policy(monkeypatch, None)
    assert pol.dense_from == radix_ops.MC_MAX + 1 == swap.GEMM_MIN_ROWS == 9
    want = {1: "gemv", 2: "mc", 5: "mc", 8: "mc", 9: "dense", 4096: "dense"}
    assert {m: pol.arm(m) for m in want} == want


def test_env_threshold_is_read_once(monkeypatch):
    pol = _policy(monkeypatch, "4")
    assert [pol.arm(m) for m in (1, 2, 3, 4, 8, 9)] == ["gemv", "mc", "mc", "dense", "dense", "dense"]
    monkeypatch.setenv(swap.ENV_DENSE_MIN, "100")
    assert pol.arm(8) == "dense"  # cached: the environment is not read again
    pol.reset()
    assert pol.arm(8) == "mc" and pol.arm(100) == "dense"


@pytest.mark.parametrize("value", ["0", "-3"])
def test_dense_arm_off(monkeypatch, value):
    pol = _policy(monkeypatch, value)
    assert [pol.arm(m) for m in (1, 2, 8, 9, 64)] == ["gemv", "mc", "mc", "loop", "loop"]


def test_unparsable_threshold_warns_and_keeps_the_default(monkeypatch):
    pol = _policy(monkeypatch, "nine")
    with pytest.warns(UserWarning, match="not an integer"):
        assert pol.dense_from == 9
    assert pol.arm(9) == "dense"


def test_threshold_one_still_sends_one_row_to_gemv(monkeypatch):
    pol = _policy(monkeypatch, "1")
    assert pol.arm(1) == "gemv" and pol.arm(2) == "dense"


def test_raw_tensor_module_is_f_linear():
    rng = np.random.default_rng(9)
    bits = (rng.integers(0x3C00, 0x3D00, (48, 64)) | (rng.integers(0, 2, (48, 64)) << 15)).astype(np.uint16)
    pack = {"codec": "raw", "R": 48, "C": 64, "raw_bits": bits}
    bias = torch.linspace(-1, 1, 48).to(torch.bfloat16)
    mod = swap.make_module(pack, bias, "cpu")
    assert isinstance(mod, swap.RawLinear) and mod.tensor_codec == "raw"
    W = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    x = torch.randn(3, 64).to(torch.bfloat16)
    assert torch.equal(mod(x), torch.nn.functional.linear(x, W, bias))


def test_make_module_refuses_other_codecs():
    with pytest.raises(ValueError, match="not a radix or raw"):
        swap.make_module({"codec": "fp8"}, None, "cpu")


def test_radix_module_refuses_a_cpu_device():
    from tests.helpers import oracle_dict

    rng = np.random.default_rng(3)
    from tests.helpers import finite_bits

    d = oracle_dict(finite_bits(rng, (8, 1024)), "sip")
    with pytest.raises(ValueError, match="GPU"):
        swap.to_device_radix(d, "cpu")


def test_to_device_raw_keeps_the_bits_in_a_copy_of_its_own():
    import numpy as np

    from drinkme_amd import radix_pack, swap

    U = np.random.default_rng(3).integers(0, 1 << 16, (6, 1024), dtype=np.uint16)
    rt = swap.to_device_raw(radix_pack.raw_dict(U), "cpu")
    assert rt["codec"] == "raw" and (rt["R"], rt["C"]) == U.shape and rt["weight"].dtype == torch.bfloat16
    got = rt["weight"].view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, U)
    U[0, 0] ^= 1
    assert got[0, 0] != U[0, 0], "the resident weight must not alias the pack's array"
