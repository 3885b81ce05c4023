"""transformer_amd -- MI355X (gfx950) Multi-Head Latent Attention hot path.

A drop-in for the MLA module of manningwu07/transformer (transformer.py:128-316):
the same ``MLA(args)`` constructor, ``forward(x, kv_cache=None, use_cache=False)``,
state-dict keys and KV-cache dict, with attention, RoPE and the absorbed decode
running as hand-written HIP kernels behind the C ABI of ``include/mla_mi355x.h``;
and a drop-in ``RMSNorm`` (transformer.py:16-27) for the block's norm1 in front of it.
"""
from . import kernels  # noqa: F401  (registers torch.ops.mla_mi355x.*)
from .config import ModelArgs  # noqa: F401
from .decode_graph import DecodeGraph  # noqa: F401
from .mla import MLA, RotaryEmbedding, apply_rope, release_decode_graphs  # noqa: F401
from .norm import RMSNorm, fused_rmsnorm_down_proj  # noqa: F401
from .ce import chunked_linear_cross_entropy  # noqa: F401

__all__ = ["MLA", "RotaryEmbedding", "apply_rope", "release_decode_graphs", "ModelArgs", "DecodeGraph", "RMSNorm", "fused_rmsnorm_down_proj",
           "chunked_linear_cross_entropy", "kernels"]
