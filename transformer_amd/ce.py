"""Vocabulary-chunked linear cross-entropy on the MI355X.

``chunked_linear_cross_entropy(x, weight_tied, targets, vocab_chunk_size=4096,
reduction="mean")`` keeps the signature and result of the reference function
(transformer.py:62-115): the exact softmax cross-entropy of ``x [B, T, D]`` against the
tied output weights ``[V, D]`` without materialising the ``[B, T, V]`` logits.

Per vocabulary chunk, hipBLASLt computes the chunk's logits in the reference's dtype (bf16
with fp32 accumulation under autocast; fp32 for an fp32 caller outside autocast, as the
reference's matmul) and one HIP kernel (``mla_ce_chunk``) folds their
fp32 log-sum-exp into the running one and gathers the target logits -- the reference
does that with ``.float()``, ``logsumexp``, ``logaddexp`` and a masked gather behind a
host sync (``in_chunk.any()``) per chunk.  The backward recomputes each chunk's logits,
turns them in place into ``g (softmax - onehot)`` with the same kernel, and accumulates
``dx += dlogits W_c`` and ``dW_c = dlogits^T x``: memory stays O(N * chunk) in training
too (the reference's autograd keeps every chunk's fp32 logits).  ``dx`` is accumulated in
fp32 across the chunks, as autograd accumulates the reference's per-chunk input gradients.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import kernels  # noqa: F401  (registers the ops)

ops = kernels.eager  # torch.ops.mla_mi355x, without the dispatcher where nothing needs it


def _compute_dtype(x: Tensor, weight: Tensor) -> torch.dtype:
    """The dtype of the reference's ``x @ w.t()`` (transformer.py:96-98): the autocast dtype
    under autocast, else the promoted dtype of x and the weights.  The kernel reads bf16 and
    fp32 logits."""
    if torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
    else:
        dt = torch.promote_types(x.dtype, weight.dtype)
    if dt not in (torch.bfloat16, torch.float32):
        raise TypeError(f"chunked_linear_cross_entropy: logits of {dt} are not built (bfloat16 under autocast, or "
                        "float32)")
    return dt


class _ChunkedCE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x2, weight, targets, chunk, reduction, cdt):
        N = x2.size(0)
        V = weight.size(0)
        xb = x2.to(cdt)
        lse = torch.full((N,), float("-inf"), dtype=torch.float32, device=x2.device)
        tl = torch.zeros(N, dtype=torch.float32, device=x2.device)
        for v0 in range(0, V, chunk):
            w = weight[v0:v0 + chunk].to(cdt)
            logits = torch.matmul(xb, w.t())  # [N, Vc] in the reference's dtype (transformer.py:96-98)
            ops.ce_chunk_fwd(logits, targets, lse, tl, v0)
        loss = lse - tl
        ctx.save_for_backward(x2, weight, targets, lse)
        ctx.chunk, ctx.reduction, ctx.cdt = chunk, reduction, cdt
        if reduction == "mean":
            return loss.mean()
        if reduction == "sum":
            return loss.sum()
        return loss

    @staticmethod
    def backward(ctx, g):
        x2, weight, targets, lse = ctx.saved_tensors
        N, V = x2.size(0), weight.size(0)
        # the upstream gradient stays on the device (no host sync): a per-row factor for the kernel
        if ctx.reduction == "mean":
            g_vec = (g.float() / max(N, 1)).expand(N).contiguous()
        elif ctx.reduction == "sum":
            g_vec = g.float().expand(N).contiguous()
        else:
            g_vec = g.reshape(N).float().contiguous()
        g_scale = 1.0
        cdt = ctx.cdt
        xb = x2.to(cdt)
        # the input gradient is summed over the chunks in fp32: each chunk's product dl W_c is
        # formed in the compute dtype (as the reference's per-chunk matmul backward) and added
        dx = torch.zeros(x2.shape, dtype=torch.float32, device=x2.device)
        dw = torch.empty(weight.shape, dtype=cdt, device=weight.device)
        for v0 in range(0, V, ctx.chunk):
            w = weight[v0:v0 + ctx.chunk].to(cdt)
            dl = torch.matmul(xb, w.t())
            ops.ce_chunk_bwd_(dl, targets, lse, g_vec, g_scale, v0)  # dl = g (softmax - onehot)
            if cdt == torch.float32:
                dx.addmm_(dl, w)
            else:
                dx.add_(torch.matmul(dl, w))
            torch.matmul(dl.t(), xb, out=dw[v0:v0 + ctx.chunk])
        return dx.to(x2.dtype), dw.to(weight.dtype), None, None, None, None


def chunked_linear_cross_entropy(x: Tensor, weight_tied: Tensor, targets: Tensor, vocab_chunk_size: int = 4096,
                                 reduction: str = "mean") -> Tensor:
    """Exact softmax CE over vocabulary chunks (transformer.py:62-115):
    ``loss_i = logsumexp_j (x_i . W_j) - x_i . W_{y_i}``, reduced by ``reduction``
    ("mean", "sum" or anything else for the per-token ``[B, T]`` losses)."""
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError("chunked_linear_cross_entropy: x must be a floating tensor")
    if weight_tied.dim() != 2 or targets.dtype != torch.long:
        raise ValueError("chunked_linear_cross_entropy: weight_tied must be [V, D] and targets long")
    if not x.is_cuda:
        raise RuntimeError("transformer_amd.chunked_linear_cross_entropy runs on a ROCm GPU only (no CPU path)")
    B, T, D = x.shape
    V = weight_tied.size(0)
    if weight_tied.size(1) != D:
        raise ValueError("chunked_linear_cross_entropy: weight_tied and x disagree on D")
    chunk = int(vocab_chunk_size)
    if chunk <= 0 or chunk % 8 or V % 8:
        raise ValueError("chunked_linear_cross_entropy: the chunk size and the vocabulary must be multiples of 8")
    yt = targets.reshape(B * T).contiguous()
    loss = _ChunkedCE.apply(x.reshape(B * T, D), weight_tied, yt, chunk, reduction, _compute_dtype(x, weight_tied))
    return loss if reduction in ("mean", "sum") else loss.view(B, T)
