"""CPU pin of the backward's rounding model (tests/gpu_util.py): with the roundings switched off
and the exact forward output it is the exact backward, fp64 autograd of the oracle attention (the
SDPA backward of transformer.py:314); with them on, its error against that backward stays within
the path's bf16 bound, so the model is a refinement of the oracle and not a different function."""
import math

import pytest
import torch

from oracle import mla_oracle as O
from tests.gpu_util import backward_rounding_model, randn_bf16
from tests.test_gpu_backward import oracle_grads
from tests.test_gpu_prefill import make_inputs, oracle

SHAPES = [
    # B, Tq, Tk, H, Hr, dn, causal, q_offset
    (1, 1, 2, 1, 1, 64, True, 1),
    (2, 40, 40, 2, 1, 128, True, 0),
    (1, 33, 70, 3, 3, 64, True, 37),
    (2, 20, 50, 2, 1, 128, False, 0),
]


@pytest.mark.parametrize("B,Tq,Tk,H,Hr,dn,causal,q_offset", SHAPES)
def test_rounding_model_without_roundings_is_the_exact_backward(B, Tq, Tk, H, Hr, dn, causal, q_offset):
    inp = make_inputs(B, Tq, Tk, H, Hr, dn, seed=Tq + Tk)
    do = randn_bf16((B, Tq, H, 128), torch.Generator().manual_seed(3))
    scale = 1 / math.sqrt(dn + 64)
    o_exact, _ = oracle(inp, scale, causal, q_offset)
    model = backward_rounding_model(inp, do, o_exact, scale, causal, q_offset, rnd=lambda t: t)
    ref = oracle_grads(inp, do, scale, causal, q_offset)
    for n in ref:
        torch.testing.assert_close(model[n], ref[n], rtol=1e-9, atol=1e-12, msg=n)


@pytest.mark.parametrize("B,Tq,Tk,H,Hr,dn,causal,q_offset", SHAPES)
def test_rounding_model_stays_within_the_bf16_bound(B, Tq, Tk, H, Hr, dn, causal, q_offset):
    inp = make_inputs(B, Tq, Tk, H, Hr, dn, seed=Tq * 3 + Tk)
    do = randn_bf16((B, Tq, H, 128), torch.Generator().manual_seed(4))
    scale = 1 / math.sqrt(dn + 64)
    o_exact, _ = oracle(inp, scale, causal, q_offset)
    model = backward_rounding_model(inp, do, o_exact.to(torch.bfloat16), scale, causal, q_offset)
    ref = oracle_grads(inp, do, scale, causal, q_offset)
    for n in ref:
        scale_n = max(1.0, ref[n].pow(2).mean().sqrt().item())
        assert (model[n] - ref[n]).abs().max().item() <= 2e-2 * scale_n, n
        assert not torch.equal(model[n], ref[n]) or ref[n].abs().max().item() == 0, f"{n}: roundings had no effect"
