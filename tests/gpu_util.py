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
