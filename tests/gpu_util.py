"""Shared helpers for the GPU parity tests (seeded CPU inputs, tolerance checks)."""
import math

import torch

from oracle import mla_oracle as O

# the parity bound of the path: bf16 output vs the fp32 (here fp64) oracle
MAX_ABS = 2e-2
MEAN_ABS = 2e-3
ROWSUM_TOL = 1e-3


def randn_bf16(shape, g, scale=1.0):
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def check_close(got: torch.Tensor, ref: torch.Tensor, what: str, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    m = O.robust_diff(ref, got.cpu())
    assert torch.isfinite(got.float()).all(), f"{what}: non-finite output"
    assert m["max"] <= max_abs and m["mean"] <= mean_abs, f"{what}: {m} (tol max {max_abs}, mean {mean_abs})"
    return m


def rowsum_from_lse(q, k, lse, scale, causal, q_offset, rows):
    """sum_j exp(s_ij - lse_i) in fp64 for the given query rows of one (b, h);
    q [Tq, D], k [Tk, D] (already concatenated nope ++ rope), lse [Tq]."""
    out = []
    for i in rows:
        s = (k.double() @ q[i].double()) * scale
        if causal:
            s[i + q_offset + 1:] = float("-inf")
        out.append(torch.exp(s - float(lse[i])).sum().item())
    return out


def _round_bf16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).to(t.dtype)


def backward_rounding_model(inp, do, o, scale, causal, q_offset, rnd=_round_bf16):
    """fp64 model of where the attention backward rounds: the flash-attention backward's placement,
    which SDPA's bf16 kernels follow for the reference's transformer.py:314.  D = rowsum(dO o O) is
    taken from the forward's bf16 output ``o [B, Tq, H, dv]``; P and dS = P (dP - D) are rounded
    (``rnd``) before the products that take them (dV = P^T dO, dQ = dS K scale, dK = dS^T Q scale);
    each gradient is rounded once (a shared k_rope head: its fp64 sum over the query heads, rounded
    once).  With ``rnd`` the identity and the exact O it is the exact backward.  Inputs as
    ``tests.test_gpu_prefill.make_inputs``; returns the five gradients in their [B, T, H, D] layouts."""
    q = torch.cat([inp["q_nope"], inp["q_rope"]], -1).double().transpose(1, 2)  # [B, H, Tq, D]
    H, dn = q.shape[1], inp["q_nope"].shape[-1]
    k = torch.cat([inp["k_nope"].double().transpose(1, 2),
                   inp["k_rope"].double().transpose(1, 2).expand(-1, H, -1, -1)], -1)
    v = inp["v"].double().transpose(1, 2)
    d_o = do.double().transpose(1, 2)
    s = q @ k.transpose(-1, -2) * scale
    if causal:  # key j is visible to query t when j <= t + q_offset
        s = s.masked_fill(~O._causal_mask(s.shape[-2], s.shape[-1], q_offset, s.device), float("-inf"))
    p = torch.softmax(s, -1)
    dd = (d_o * o.double().transpose(1, 2)).sum(-1, keepdim=True)
    ds = p * (d_o @ v.transpose(-1, -2) - dd)
    dv = rnd(p).transpose(-1, -2) @ d_o
    dq = rnd(ds) @ k * scale
    dk = rnd(ds).transpose(-1, -2) @ q * scale
    dq, dk, dv = (t.transpose(1, 2) for t in (dq, dk, dv))
    dkr = dk[..., dn:]
    if inp["k_rope"].shape[2] == 1:
        dkr = dkr.sum(2, keepdim=True)
    out = dict(dq_nope=dq[..., :dn], dq_rope=dq[..., dn:], dk_nope=dk[..., :dn], dk_rope=dkr, dv=dv)
    return {n: rnd(t) for n, t in out.items()}
