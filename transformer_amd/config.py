"""Model arguments read by the MLA module.

Field names follow the reference's ``ModelArgs`` (params.py:14-60) so either
dataclass can be passed to :class:`transformer_amd.MLA`.  Four optional fields
generalise the head layout; left at ``None`` they reproduce the reference module
exactly (content dim = head_dim - 64, V dim = head_dim, one k_rope per head).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional


@dataclass
class ModelArgs:
    d_model: int = 1792
    n_layers: int = 28
    n_heads: int = 14
    head_dim: int = 128
    d_latent: int = 384
    q_lora_rank: int = 384
    vocab_size: int = 32768
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    hidden_size: int = 4608
    max_seq_len: int = 8192
    # MLA head layout (None => the reference's derived value)
    qk_nope_dim: Optional[int] = None     # head_dim - 64
    qk_rope_dim: int = 64
    v_head_dim: Optional[int] = None      # head_dim
    n_k_rope_heads: Optional[int] = None  # n_heads (per-head k_rope); 1 => shared k_rope

    @staticmethod
    def mla_baseline(**over) -> "ModelArgs":
        """The dims every benchmark config is quoted on: d_model 2048, 16 heads,
        q_lora 1024, kv_lora 512, qk_nope 128 + rope 64 (theta 1e4), v 128, shared
        k_rope, RoPE table long enough for T = 16384."""
        kw = dict(d_model=2048, n_heads=16, head_dim=192, d_latent=512, q_lora_rank=1024, qk_nope_dim=128,
                  qk_rope_dim=64, v_head_dim=128, n_k_rope_heads=1, rope_theta=10000.0, max_seq_len=16384)
        kw.update(over)
        return ModelArgs(**kw)


def mla_dims(args):
    """(n_heads, qk_nope, qk_rope, v_head, n_k_rope_heads) of any ModelArgs-like object."""
    H = int(args.n_heads)
    rope = int(getattr(args, "qk_rope_dim", 64) or 64)
    nope = getattr(args, "qk_nope_dim", None)
    nope = int(args.head_dim) - rope if nope is None else int(nope)
    v = getattr(args, "v_head_dim", None)
    v = int(args.head_dim) if v is None else int(v)
    hr = getattr(args, "n_k_rope_heads", None)
    hr = H if hr is None else int(hr)
    if hr not in (1, H):
        raise ValueError(f"n_k_rope_heads must be 1 or n_heads ({H}), got {hr}")
    return H, nope, rope, v, hr
