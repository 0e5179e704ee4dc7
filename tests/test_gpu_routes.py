"""GPU: the served module's M routes (src/drinkme/codec/swap.py:302-335,
:340-392) over the C ABI.

  - M = 1 "gemv" and 2..8 "mc": fp32 accumulation, bias in fp32, one
    rounding to x's dtype; within the float64 bound;
  - M >= 9 "dense": the weight decoded once (exact bits) and the same
    F.linear stock runs, so the output equals F.linear over the source
    weight bit for bit (swap.py:361-375);
  - M > 8 with the dense arm disabled (DRINKME_PREFILL_DENSE_MIN = 0):
    "loop", one GEMV per row.
"""

import numpy as np
import pytest

from oracle import radix_oracle as O
from tests.helpers import bf16_tensor, finite_bits, oracle_dict

pytestmark = pytest.mark.gpu


@pytest.fixture
def module(cuda):
    import torch

    from drinkme_amd import swap

    rng = np.random.default_rng(123)
    bits = finite_bits(rng, (640, 2048))
    bias_bits = O.f32_to_bf16_bits(rng.standard_normal(640).astype(np.float32) * 0.1)
    bias = bf16_tensor(bias_bits, cuda)
    mod = swap.make_module(oracle_dict(bits, "sip"), bias, cuda)
    W = bf16_tensor(bits, cuda)
    return mod, W, bias, rng, torch


@pytest.mark.parametrize("M", [1, 2, 5, 8])
def test_gemv_and_mc_routes(module, M):
    mod, W, bias, rng, torch = module
    x = torch.from_numpy(rng.standard_normal((M, 2048)).astype(np.float32)).to(W.device).to(torch.bfloat16)
    assert mod._route(x) == ("gemv" if M == 1 else "mc")
    y = mod(x)
    assert y.dtype == torch.bfloat16 and y.shape == (M, 640)
    ref = torch.nn.functional.linear(x.float(), W.float(), bias.float())
    err = (y.float() - ref).abs()
    # one bf16 rounding of a float64-accurate result: half an ulp plus the bound
    assert torch.all(err <= ref.abs() * 2 ** -8 + 1e-3)


def test_dense_route_is_stock_f_linear_bit_for_bit(module):
    mod, W, bias, rng, torch = module
    x = torch.from_numpy(rng.standard_normal((2, 9, 2048)).astype(np.float32)).to(W.device).to(torch.bfloat16)
    assert mod._route(x) == "dense"
    y = mod(x)
    assert torch.equal(y, torch.nn.functional.linear(x, W, bias))


def test_loop_route_when_the_dense_arm_is_disabled(module, monkeypatch):
    mod, W, bias, rng, torch = module
    from drinkme_amd import swap

    monkeypatch.setattr(swap.ROUTES, "_dense_from", 0)
    x = torch.from_numpy(rng.standard_normal((12, 2048)).astype(np.float32)).to(W.device).to(torch.bfloat16)
    assert mod._route(x) == "loop"
    y = mod(x)
    ref = torch.nn.functional.linear(x.float(), W.float(), bias.float())
    assert torch.all((y.float() - ref).abs() <= ref.abs() * 2 ** -7 + 1e-3)


def test_cpu_input_is_refused(module):
    mod, W, bias, rng, torch = module
    with pytest.raises(RuntimeError, match="GPU"):
        mod(torch.zeros(1, 2048, dtype=torch.bfloat16))
