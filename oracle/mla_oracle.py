"""CPU oracle for the MLA hot path -- TEST INFRASTRUCTURE ONLY.

This module is a plain PyTorch-CPU restatement of the reference's Multi-Head
Latent Attention path (manningwu07/transformer, ``transformer.py``).  It exists
to *check* the HIP kernels in ``transformer_amd`` and to time a CPU baseline.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import it; the product package never does, and there is no CPU
fallback in the product path.

Every function cites the reference lines it restates.  Generalised dims
(``qk_nope_dim``, ``qk_rope_dim``, ``v_head_dim``, ``n_k_rope_heads``) reduce to
the reference module when ``v_head_dim == qk_nope_dim + qk_rope_dim`` and
``n_k_rope_heads == n_heads``.

How each function is pinned (tests/test_oracle.py):
  rope_tables      -- golden vectors written by the reference itself
                      (tests/golden/mla_ref_golden.npz) and the fp64 closed
                      form cos/sin(p * theta^(-2i/d)) within one bf16 ulp.
  apply_rope       -- complex-multiplication form (x1 + i x2) * e^{i phi},
                      norm preservation, exact inverse, and position-shift
                      invariance <R_p q, R_p' k> = <q, R_(p'-p) k>.
  attention        -- torch CPU scaled_dot_product_attention (a library
                      routine), fp64 brute-force loops on tiny shapes, rows of
                      P summing to 1, V = ones => O = 1, O[0] = V[0] (causal),
                      prefix independence and the reference's own
                      triu(diagonal=pos_offset+1) mask construction.
  attention_bwd    -- torch.autograd.gradcheck (finite differences) on tiny
                      fp64 shapes, SDPA autograd, and sum_j dS_ij = 0.
  absorbed_decode  -- algebraic equality with the non-absorbed attention by
                      linearity (also with the chunk mask: q_offset), L = 1 =>
                      ctx = c_0, split-K LSE merge equal to the full softmax,
                      and each query of a masked chunk equal to a one-query
                      call over its visible prefix.
  rms_norm         -- torch.nn.functional.rms_norm (a library routine) in fp64,
                      constant rows (closed form), mean(y^2 / w^2) = 1 and scale
                      invariance at eps = 0.
  rms_norm_bwd     -- torch.autograd.gradcheck and sum_k x_k dx_k = 0 at eps = 0
                      (the norm is invariant to the scale of its row).
  rmsnorm_down_proj -- identity w_down gives the bf16 norm itself; exact tiny cases
                      (rows of equal magnitude) and the reference's rsqrt form.
  chunked_linear_cross_entropy -- torch.nn.functional.cross_entropy on the full
                      logits (a library routine), chunk-size invariance, zero
                      weights => log V, torch.autograd.gradcheck.
  mla_forward      -- golden vectors of the reference MLA module (both
                      branches, prefill + decode with cache, reference dims),
                      and decode-after-prefill == no-cache forward on the
                      concatenated sequence.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import torch
import torch.nn.functional as F

__all__ = [
    "MLADims",
    "rms_norm",
    "rms_norm_bwd",
    "rmsnorm_down_proj",
    "chunked_linear_cross_entropy",
    "rope_tables",
    "apply_rope",
    "attention",
    "attention_bwd",
    "absorbed_decode",
    "merge_splits",
    "init_weights",
    "mla_forward",
    "robust_diff",
]

LOG2E = 1.4426950408889634


@dataclass
class MLADims:
    """Dims of one MLA layer.

    Reference fields: ``transformer.py:133-170`` and ``params.py:17-36``
    (``n_heads``, ``head_dim``, ``d_model``, ``q_lora_rank``, ``d_latent``,
    ``rope_theta``, ``max_seq_len``).  The reference fixes rope_dim = 64
    (``transformer.py:138``) and derives content dim = head_dim - 64
    (``:141``) and v dim = head_dim (``:160``); the generalised fields below
    default to exactly that.
    """

    d_model: int = 2048
    n_heads: int = 16
    q_lora_rank: int = 1024
    d_latent: int = 512
    qk_nope_dim: int = 128
    qk_rope_dim: int = 64
    v_head_dim: int = 128
    n_k_rope_heads: int = 1
    rope_theta: float = 10000.0
    max_seq_len: int = 16384
    rms_norm_eps: float = 1e-6

    @property
    def d_qk(self) -> int:
        return self.qk_nope_dim + self.qk_rope_dim

    @property
    def scale(self) -> float:
        # transformer.py:170 (absorbed branch) and SDPA's default 1/sqrt(q.size(-1))
        # at transformer.py:314 -- both are 1/sqrt(d_qk).
        return 1.0 / math.sqrt(self.d_qk)

    @staticmethod
    def reference(d_model=1792, n_heads=14, head_dim=128, d_latent=384, q_lora_rank=None,
                  rope_theta=10000.0, max_seq_len=8192) -> "MLADims":
        """The reference module's own dims (params.py:17-36; q_lora_rank = d_latent, :24)."""
        return MLADims(d_model=d_model, n_heads=n_heads,
                       q_lora_rank=d_latent if q_lora_rank is None else q_lora_rank,
                       d_latent=d_latent, qk_nope_dim=head_dim - 64, qk_rope_dim=64,
                       v_head_dim=head_dim, n_k_rope_heads=n_heads,
                       rope_theta=rope_theta, max_seq_len=max_seq_len)


def rms_norm(x: torch.Tensor, weight: Optional[torch.Tensor] = None, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm, transformer.py:16-27: ``x * rsqrt(mean(x^2) + eps) * weight`` in x's dtype
    (the block's norm1 in front of the down-projections, transformer.py:338)."""
    y = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return y if weight is None else y * weight


def rms_norm_bwd(x: torch.Tensor, weight: torch.Tensor, dy: torch.Tensor, eps: float = 1e-6,
                 dtype=torch.float64):
    """(dx, dw) of :func:`rms_norm` by autograd in ``dtype`` (the backward PyTorch runs for
    transformer.py:26-27)."""
    xx = x.to(dtype).detach().requires_grad_(True)
    ww = weight.to(dtype).detach().requires_grad_(True)
    y = rms_norm(xx, ww, eps)
    dx, dw = torch.autograd.grad(y, (xx, ww), dy.to(dtype))
    return dx, dw


def rmsnorm_down_proj(x: torch.Tensor, w_norm: torch.Tensor, w_down: torch.Tensor, eps: float = 1e-6):
    """The reference's baseline for its fused RMSNorm + down-projection kernel
    (fused_mla_triton_kernels.py:813-816): fp32 ``x / sqrt(mean(x^2) + eps) * w_norm``,
    rounded to bf16, times ``w_down [K, N]`` with fp32 accumulation, rounded to bf16."""
    xf = x.float()
    rms = torch.sqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    xn = ((xf / rms) * w_norm.float()).to(torch.bfloat16)
    return (xn.float() @ w_down.float()).to(torch.bfloat16)


def chunked_linear_cross_entropy(x: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                                 vocab_chunk_size: int = 4096, reduction: str = "mean", dtype=torch.float64):
    """transformer.py:62-115 in ``dtype``: per vocabulary chunk, logits = x W_c^T, the running
    lse = logaddexp(lse, logsumexp(logits)) and the target logit when it lies in the chunk;
    loss = lse - target logit, reduced by ``reduction``."""
    B, T, D = x.shape
    xt = x.reshape(B * T, D).to(dtype)
    yt = targets.reshape(B * T)
    lse = torch.full((B * T,), float("-inf"), dtype=dtype)
    tl = torch.zeros(B * T, dtype=dtype)
    for v0 in range(0, weight.size(0), vocab_chunk_size):
        v1 = min(weight.size(0), v0 + vocab_chunk_size)
        logits = xt @ weight[v0:v1].to(dtype).t()
        lse = torch.logaddexp(lse, torch.logsumexp(logits, dim=-1))
        m = (yt >= v0) & (yt < v1)
        tl[m] = logits[m, (yt[m] - v0)]
    loss = lse - tl
    if reduction == "mean":
        return loss.mean()
    if reduction == "sum":
        return loss.sum()
    return loss.view(B, T)


def rope_tables(rope_dim: int = 64, max_seq_len: int = 8192, theta: float = 10000.0
                ) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables ``[max_seq_len, rope_dim/2]`` rounded to bf16.

    transformer.py:29-44: inv_freq_i = theta^(-2i/d) in fp32, angle = t * inv_freq
    (fp32 outer product), cos/sin evaluated in fp32 and stored as bf16 even for fp32
    runs (they are cast back to x.dtype at use, :50-52).
    """
    freqs = 1.0 / (theta ** (torch.arange(0, rope_dim, 2).float() / rope_dim))
    t = torch.arange(max_seq_len)
    ang = torch.outer(t, freqs).float()
    return ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Split-half rotation of the last dim, transformer.py:55-60.

    ``x[..., T, d]``; ``cos``/``sin`` broadcast as ``[T, d/2]``.
    y1 = x1 c - x2 s ; y2 = x1 s + x2 c.
    """
    cos = cos.to(x.dtype)
    sin = sin.to(x.dtype)
    d = x.shape[-1] // 2
    x1, x2 = x[..., :d], x[..., d:]
    return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1)


def _causal_mask(tq: int, tk: int, q_offset: int, device=None) -> torch.Tensor:
    """Boolean mask, True where key j is visible to query i: j <= i + q_offset.

    Equivalent to the reference's additive mask ``triu(full(-inf), diagonal=pos_offset+1)``
    (transformer.py:273-281) and to SDPA's ``is_causal`` for tq == tk, q_offset == 0
    (transformer.py:314).
    """
    i = torch.arange(tq, device=device).unsqueeze(1)
    j = torch.arange(tk, device=device).unsqueeze(0)
    return j <= i + q_offset


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
              causal: bool = True, q_offset: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """O = softmax(Q K^T * scale + M) V and the natural-log LSE of each row.

    ``q [..., Tq, Dqk]``, ``k [..., Tk, Dqk]``, ``v [..., Tk, Dv]`` (leading dims
    broadcast, e.g. a shared k_rope head).  This is what
    ``F.scaled_dot_product_attention(q, k, v, is_causal=True)`` computes at
    transformer.py:314, with the bottom-right offset of the absorbed prefill mask
    (transformer.py:273-281) as ``q_offset``.
    """
    s = torch.matmul(q, k.transpose(-1, -2)) * scale
    if causal:
        m = _causal_mask(q.shape[-2], k.shape[-2], q_offset, q.device)
        s = s.masked_fill(~m, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.exp(s - lse.unsqueeze(-1))
    return torch.matmul(p, v), lse


def attention_bwd(q, k, v, do, scale, causal=True, q_offset=0, dtype=torch.float64):
    """dQ, dK, dV of :func:`attention` by autograd (the reference's backward is SDPA's
    autograd through transformer.py:314)."""
    qq = q.detach().to(dtype).requires_grad_(True)
    kk = k.detach().to(dtype).requires_grad_(True)
    vv = v.detach().to(dtype).requires_grad_(True)
    o, _ = attention(qq, kk, vv, scale, causal, q_offset)
    dq, dk, dv = torch.autograd.grad(o, (qq, kk, vv), do.to(dtype))
    return dq, dk, dv


def absorbed_decode(q_lat, q_rope, c_kv, k_rope, scale, seq_lens=None, q_offset=None):
    """Absorbed latent attention, transformer.py:249-286.

    ``q_lat [B,H,T,DL]`` (= q_nope . W_UK, :252-254), ``q_rope [B,H,T,R]``,
    ``c_kv [B,L,DL]`` (shared by all heads, :257), ``k_rope [B,Hr,L,R]`` (Hr = 1 or H).
    scores = (q_lat c^T + q_rope k_rope^T) * scale (:259-269); softmax (:283);
    ctx = P c (:286).  ``seq_lens`` (optional, per batch) masks keys >= seq_len;
    ``q_offset`` (optional) applies the reference's chunk mask triu(diagonal=pos_offset+1)
    (:273-281): query t sees keys j <= t + q_offset.
    Returns ``ctx [B,H,T,DL]`` and ``lse [B,H,T]``.
    """
    lat = c_kv.unsqueeze(1)
    s = torch.matmul(q_lat, lat.transpose(-1, -2)) + torch.matmul(q_rope, k_rope.transpose(-1, -2))
    s = s * scale
    if q_offset is not None:
        s = s.masked_fill(~_causal_mask(s.shape[-2], s.shape[-1], q_offset, s.device), float("-inf"))
    if seq_lens is not None:
        L = c_kv.shape[1]
        valid = torch.arange(L).unsqueeze(0) < torch.as_tensor(seq_lens).view(-1, 1)
        s = s.masked_fill(~valid[:, None, None, :], float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.exp(s - lse.unsqueeze(-1))
    return torch.matmul(p, lat), lse


def merge_splits(ctx_parts: torch.Tensor, lse_parts: torch.Tensor):
    """Merge normalised partial results of disjoint key ranges (split-K).

    ``ctx_parts [S, ...,  D]`` each normalised over its own keys, ``lse_parts [S, ...]``.
    lse = log sum_s exp(lse_s) ; ctx = sum_s exp(lse_s - lse) ctx_s.
    """
    lse = torch.logsumexp(lse_parts, dim=0)
    w = torch.exp(lse_parts - lse.unsqueeze(0))
    w = torch.nan_to_num(w, nan=0.0)
    return (w.unsqueeze(-1) * ctx_parts).sum(0), lse


def init_weights(dims: MLADims, generator: torch.Generator, std: float = 0.02,
                 dtype=torch.float32) -> Dict[str, torch.Tensor]:
    """Seeded N(0, std) weights in module registration order (transformer.py:145-163,
    init as transformer.py:450-454).  Keys match the reference state dict."""
    H, dn, dr, dv, Hr = dims.n_heads, dims.qk_nope_dim, dims.qk_rope_dim, dims.v_head_dim, dims.n_k_rope_heads
    shapes = [
        ("q_down.weight", (dims.q_lora_rank, dims.d_model)),
        ("q_up.weight", (H * dn, dims.q_lora_rank)),
        ("qk_rope.weight", ((H + Hr) * dr, dims.d_model)),
        ("kv_down.weight", (dims.d_latent, dims.d_model)),
        ("k_up.weight", (H * dn, dims.d_latent)),
        ("v_up.weight", (H * dv, dims.d_latent)),
        ("o_proj.weight", (dims.d_model, H * dv)),
    ]
    return {name: (torch.randn(shape, generator=generator) * std).to(dtype) for name, shape in shapes}


def mla_forward(w: Dict[str, torch.Tensor], x: torch.Tensor, dims: MLADims,
                kv_cache: Optional[dict] = None, use_cache: bool = False,
                tables: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                dtype=torch.float64):
    """``MLA.forward(x, kv_cache, use_cache)``, transformer.py:202-316, computed in ``dtype``.

    Returns ``(out [B,T,d_model], new_cache | None)`` with the reference's cache dict
    ``{"latent": [B,L,DL], "k_rope": [B,Hr,L,R] post-RoPE, "seq_len": L}``.
    """
    H, dn, dr, dv, Hr = dims.n_heads, dims.qk_nope_dim, dims.qk_rope_dim, dims.v_head_dim, dims.n_k_rope_heads
    B, T, _ = x.shape
    x = x.to(dtype)
    W = {k: t.to(dtype) for k, t in w.items()}
    lin = lambda t, name: t @ W[name].t()  # nn.Linear without bias

    pos_offset = kv_cache["seq_len"] if kv_cache is not None else 0  # :205
    q_content = lin(lin(x, "q_down.weight"), "q_up.weight")  # :208
    qk_pos = lin(x, "qk_rope.weight")  # :209
    q_pos, k_pos_new = qk_pos[..., : H * dr], qk_pos[..., H * dr:]  # :210 (chunk(2) when Hr == H)
    kv_new = lin(x, "kv_down.weight")  # :213
    kv_latent = torch.cat([kv_cache["latent"].to(dtype), kv_new], 1) if kv_cache is not None else kv_new  # :215-218

    q_content = q_content.view(B, T, H, dn).transpose(1, 2)  # :221
    q_pos = q_pos.view(B, T, H, dr).transpose(1, 2)  # :222
    kv_len = kv_latent.size(1)
    if tables is None:
        tables = rope_tables(dr, max(dims.max_seq_len, kv_len), dims.rope_theta)
    cos, sin = tables[0][:kv_len], tables[1][:kv_len]  # :228
    c, s = cos[pos_offset:pos_offset + T], sin[pos_offset:pos_offset + T]  # :231-232
    q_pos = apply_rope(q_pos, c, s)  # :233
    k_pos_new = apply_rope(k_pos_new.view(B, T, Hr, dr).transpose(1, 2), c, s)  # :236-239
    k_pos = torch.cat([kv_cache["k_rope"].to(dtype), k_pos_new], 2) if kv_cache is not None else k_pos_new  # :241-244

    scale = dims.scale
    if use_cache:  # absorbed branch, :249-300
        Wk = W["k_up.weight"].view(H, dn, -1)
        q_lat = torch.einsum("bhtc,hcd->bhtd", q_content, Wk)  # :252-254
        # the reference masks for every T > 1 (and T == 1 without cache, where it is a no-op)
        s_ = (torch.matmul(q_lat, kv_latent.unsqueeze(1).transpose(-1, -2))
              + torch.matmul(q_pos, k_pos.transpose(-1, -2))) * scale  # :259-269
        m = _causal_mask(T, kv_len, pos_offset)
        s_ = s_.masked_fill(~m, float("-inf"))  # :273-281
        p = torch.softmax(s_, dim=-1)  # :283
        ctx = torch.matmul(p, kv_latent.unsqueeze(1))  # :286
        Wv = W["v_up.weight"].view(H, dv, -1)
        out = torch.einsum("bhtd,hmd->bhtm", ctx, Wv)  # :290-291
        out = out.transpose(1, 2).reshape(B, T, H * dv)
        cache = {"latent": kv_latent, "k_rope": k_pos, "seq_len": kv_len}  # :295-299
        return lin(out, "o_proj.weight"), cache

    # training / no-cache branch, :306-316
    k_content = lin(kv_latent, "k_up.weight").view(B, kv_len, H, dn).transpose(1, 2)  # :307
    v = lin(kv_latent, "v_up.weight").view(B, kv_len, H, dv).transpose(1, 2)  # :308
    q = torch.cat([q_content, q_pos], -1)  # :311 (rope last)
    k = torch.cat([k_content, k_pos.expand(B, H, kv_len, dr)], -1)  # :312
    o, _ = attention(q, k, v, scale, causal=True, q_offset=0)  # :314 (is_causal, top-left)
    o = o.transpose(1, 2).reshape(B, T, H * dv)  # :315
    return lin(o, "o_proj.weight"), None


def robust_diff(expected: torch.Tensor, actual: torch.Tensor) -> Dict[str, float]:
    """mean / p99 / p999 / max abs difference, the reporting shape of
    fused_mla_triton_kernels.py:72-80."""
    d = (expected.double() - actual.double()).abs().flatten()
    n = d.numel()
    if n == 0:
        return {"mean": 0.0, "p99": 0.0, "p999": 0.0, "max": 0.0}
    srt = torch.sort(d).values
    return {
        "mean": float(d.mean()),
        "p99": float(srt[max(0, int(0.99 * n) - 1)]),
        "p999": float(srt[max(0, int(0.999 * n) - 1)]),
        "max": float(srt[-1]),
    }
