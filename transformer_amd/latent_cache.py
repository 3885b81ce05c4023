"""Preallocated storage behind MLA's KV-cache dict.

The reference grows its cache with ``torch.cat`` on every call (transformer.py:215-218
for the latent, :241-244 for the post-RoPE k_rope): a decode step copies the whole
cache, O(L) bytes per token per layer, more than the attention itself reads.

Here the dict keeps the reference's format, ``{"latent": [B, L, d_latent],
"k_rope": [B, Hr, L, 64], "seq_len": L}``, but its two tensors are views of the first L
positions of buffers with spare capacity.  An append writes only the new tokens.

Rules that keep the reference's value semantics:
  * an append happens in place only when the dict passed in is the newest one made
    from its buffers (``seq_len`` equals the buffers' committed length).  Any other
    dict (an older one being branched from, a cache made elsewhere, a different batch
    size or dtype) is copied into fresh buffers first, so no dict a caller holds ever
    changes under it;
  * capacity grows by 1.5x (rounded up to 256 tokens, capped at ``max_len``), so a
    sequence of appends costs amortised O(new tokens);
  * buffers are used only with autograd off (``torch.no_grad()`` or inference mode):
    with autograd on, the caller's graph may hold views of the cache, and an in-place
    append would invalidate them.  That case keeps the functional ``torch.cat`` path.

The views are not contiguous in the batch dimension (their batch stride is the
capacity); every kernel of this package takes strides.
"""
from __future__ import annotations

from typing import Optional

import torch

_ATTR = "_mla_latent_store"
_ROUND = 256


def grown_capacity(need: int, max_len: int) -> int:
    """Capacity for ``need`` tokens: 1.5x, rounded up to 256, at most ``max_len`` (>= need)."""
    if need < 0:
        raise ValueError("grown_capacity: need must be >= 0")
    cap = max(need + need // 2, need + 1)
    cap = (cap + _ROUND - 1) // _ROUND * _ROUND
    return max(need, min(cap, max_len))


class LatentCacheStore:
    """Buffers ``latent [B, C, d_latent]`` and ``k_rope [B, Hr, C, d_rope]`` with ``length``
    committed positions."""

    def __init__(self, B: int, Hr: int, d_latent: int, d_rope: int, capacity: int, dtype, device):
        self.latent = torch.empty(B, capacity, d_latent, dtype=dtype, device=device)
        self.k_rope = torch.empty(B, Hr, capacity, d_rope, dtype=dtype, device=device)
        self.length = 0

    @property
    def capacity(self) -> int:
        return self.latent.size(1)

    def fits(self, B: int, Hr: int, d_latent: int, d_rope: int, dtype, need: int) -> bool:
        return (self.latent.size(0) == B and self.latent.size(2) == d_latent and self.k_rope.size(1) == Hr
                and self.k_rope.size(3) == d_rope and self.latent.dtype == dtype and need <= self.capacity
                and (torch.is_inference_mode_enabled() or not self.latent.is_inference()))

    def views(self, n: int):
        return self.latent[:, :n], self.k_rope[:, :, :n]


def store_of(cache: Optional[dict]) -> Optional[LatentCacheStore]:
    """The store whose newest dict is ``cache``, or None (no store, or an older dict)."""
    if cache is None:
        return None
    lat = cache.get("latent")
    store = getattr(lat, _ATTR, None)
    if store is None or int(cache["seq_len"]) != store.length:
        return None
    kr = cache.get("k_rope")
    if (lat.data_ptr() != store.latent.data_ptr() or lat.stride() != store.latent.stride()
            or kr is None or kr.data_ptr() != store.k_rope.data_ptr() or kr.stride() != store.k_rope.stride()):
        return None
    return store


def reserve(cache: Optional[dict], B: int, T: int, Hr: int, d_latent: int, d_rope: int, dtype, device,
            max_len: int):
    """The store that will hold ``cache`` plus T new positions, and the first new position
    L0: ``cache`` itself when it is its store's newest dict and fits, else fresh buffers
    holding a copy of its L0 positions.  The caller writes positions [L0, L0 + T) (for
    instance with the rope_append kernel) and then calls :func:`commit`.  Must be called
    with autograd off."""
    if torch.is_grad_enabled():
        raise RuntimeError("latent_cache: call with autograd off (torch.no_grad or inference mode)")
    L0 = int(cache["seq_len"]) if cache is not None else 0
    need = L0 + T
    if need > max_len:
        raise ValueError(f"latent_cache: {need} positions exceed the limit of {max_len}")
    store = store_of(cache)
    if store is None or not store.fits(B, Hr, d_latent, d_rope, dtype, need):
        fresh = LatentCacheStore(B, Hr, d_latent, d_rope, grown_capacity(need, max_len), dtype, device)
        if L0 > 0:
            src = store.views(L0) if store is not None else (cache["latent"], cache["k_rope"])
            fresh.latent[:, :L0].copy_(src[0])
            fresh.k_rope[:, :, :L0].copy_(src[1])
        store = fresh
    return store, L0


def commit(store: LatentCacheStore, length: int):
    """Mark ``length`` positions of ``store`` as written and return ``(latent, k_rope,
    new_cache)``: views of all of them and the reference's dict format."""
    store.length = length
    latent, k_rope = store.views(length)
    out_latent = latent.detach()
    setattr(out_latent, _ATTR, store)
    return latent, k_rope, {"latent": out_latent, "k_rope": k_rope.detach(), "seq_len": length}


def append(cache: Optional[dict], latent_new: torch.Tensor, k_rope_new: torch.Tensor, max_len: int):
    """Append ``latent_new [B, T, d_latent]`` and ``k_rope_new [B, Hr, T, d_rope]`` to ``cache``
    (None for an empty one) and return ``(latent, k_rope, new_cache)``: the first two are
    views of all L + T positions; the dict is the reference's format.  Must be called with
    autograd off."""
    B, T, DL = latent_new.shape
    Hr, dr = k_rope_new.size(1), k_rope_new.size(3)
    store, L0 = reserve(cache, B, T, Hr, DL, dr, latent_new.dtype, latent_new.device, max_len)
    store.latent[:, L0:L0 + T].copy_(latent_new)
    store.k_rope[:, :, L0:L0 + T].copy_(k_rope_new)
    return commit(store, L0 + T)
