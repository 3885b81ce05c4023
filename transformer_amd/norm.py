"""RMSNorm in front of the MLA down-projections, on the MI355X.

``RMSNorm`` is a drop-in for the reference's ``RMSNorm`` (transformer.py:16-27): the same
constructor ``RMSNorm(dim, eps=1e-6)`` and ``weight`` parameter (state-dict key
``weight``).  Its forward is one HIP kernel (``mla_mi355x::rmsnorm``): one read of the
row, one bf16 write, with the fp32 arithmetic of ``x * rsqrt(mean(x^2) + eps) * weight``;
its backward is a second HIP kernel.  Used as the block's ``norm1``, it feeds ``MLA``,
which runs ``q_down``, ``qk_rope`` and ``kv_down`` as one GEMM over the concatenated
weights (one pass over the normalised rows instead of three).

The output is bf16 when x is bf16 or bf16 autocast is on: that is exactly what the
reference's down-projection GEMMs read under ``torch.autocast(bf16)`` (train.py:437),
since autocast casts the fp32 norm output to bf16 there.  Outside autocast an fp32 x
gets the fp32 result, as the reference computes it (the kernel writes fp32 rows).

``fused_rmsnorm_down_proj(x, w_norm, w_down, eps)`` keeps the signature of the
reference's fused kernel wrapper (fused_mla_triton_kernels.py:233-274; ``w_down`` is
``[K, N]``): the HIP norm kernel, then the down-projection on hipBLASLt.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import kernels  # noqa: F401  (registers the ops)

ops = kernels.eager  # torch.ops.mla_mi355x, without the dispatcher where nothing needs it


def _out_dtype(x: torch.Tensor) -> torch.dtype:
    """bf16 for bf16 rows or under bf16 autocast, else fp32 (the kernel reads bf16 and fp32 rows)."""
    if x.dtype == torch.bfloat16:
        return torch.bfloat16
    if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
        return torch.bfloat16
    return torch.float32


class RMSNorm(nn.Module):
    """RMSNorm (transformer.py:16-27) as one HIP kernel on the GPU."""

    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x):
        if not x.is_cuda:
            raise RuntimeError("transformer_amd.RMSNorm runs on a ROCm GPU only (no CPU path)")
        y, _ = ops.rmsnorm(x, self.weight, float(self.eps), _out_dtype(x) == torch.float32)
        return y


def fused_rmsnorm_down_proj(x: torch.Tensor, w_norm: torch.Tensor, w_down: torch.Tensor,
                            eps: float = 1e-6) -> torch.Tensor:
    """``bf16(bf16(rmsnorm(x) * w_norm) @ w_down)`` for ``x [M, K]`` bf16, ``w_norm [K]``,
    ``w_down [K, N]`` (the reference wrapper's layout and result,
    fused_mla_triton_kernels.py:233-274 and its test baseline :813-816).  Any K that is
    a multiple of 8 up to 4096 and any N are accepted (the reference asserts K = 1792,
    N = 384)."""
    if x.dim() != 2 or w_down.dim() != 2 or w_down.size(0) != x.size(1) or w_norm.shape != (x.size(1),):
        raise ValueError(f"fused_rmsnorm_down_proj: expected x [M, K], w_norm [K], w_down [K, N]; got "
                         f"{tuple(x.shape)}, {tuple(w_norm.shape)}, {tuple(w_down.shape)}")
    xn, _ = ops.rmsnorm(x, w_norm, float(eps))
    return torch.matmul(xn, w_down.to(torch.bfloat16))
