"""Drop-in ``MLA`` module for manningwu07/transformer (transformer.py:128-316).

Same constructor (``MLA(args)``), same ``forward(x, kv_cache=None, use_cache=False)
-> (out, new_cache)``, same parameter names / state-dict keys, the same legacy
``q_rope``/``k_rope`` -> ``qk_rope`` load hook, and the same KV-cache dict
``{"latent": [B, L, d_latent], "k_rope": [B, Hr, L, 64] post-RoPE, "seq_len": L}``.

The projections stay ``nn.Linear`` (hipBLASLt through torch).  RoPE, attention and
the absorbed decode are HIP kernels (``torch.ops.mla_mi355x``):

  no cache / training  ->  rope (q and k heads in one pass) -> prefill_fwd (causal,
                           nope/rope passed separately, no concat) ; backward via
                           prefill_bwd + rope(inverse)
  use_cache, T == 1    ->  rope -> q_lat = q_nope W_UK -> decode over the latent cache,
                           with ctx W_UV^T in its split merge; with autograd off and
                           bf16 products, the down-projections, q_up, the W_UK
                           absorption and o_proj run as few-row products (linear_rows),
                           and with bf16 weights the whole step replays a HIP graph
                           recorded against the cache's buffers (AUTO_GRAPH)
  use_cache, T > 1     ->  rope -> prefill_fwd with q_offset = pos_offset over
                           k_up/v_up of the whole latent cache (the bottom-right mask
                           of transformer.py:273-281)

With autograd off, the cache dict's tensors are views of preallocated buffers
(``latent_cache``): an append writes only the new tokens instead of the reference's
O(L) ``torch.cat``; in bf16 the RoPE kernel itself writes them (``rope_append``).  With autograd on, the cache grows by ``torch.cat`` as in the
reference.

Attention runs in bf16 (fp32 accumulation); under ``torch.autocast(bf16)`` that is
the projections' own dtype.  Tensors on the CPU raise: there is no CPU path.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn

from . import kernels  # noqa: F401  (registers the ops)
from . import latent_cache
from .decode_graph import DecodeGraph, autocast_bf16
from .config import mla_dims

ops = kernels.eager  # torch.ops.mla_mi355x, without the dispatcher where nothing needs it

# With autograd off and bf16 projections, the cache path writes the new positions with the
# RoPE kernel itself (rope_append) instead of RoPE followed by two copies; False keeps the
# latter (both give bitwise-equal caches and outputs).
ROPE_APPEND = True

# In the no-cache (training) branch with bf16 projections, the q heads' RoPE runs inside the
# attention kernel's Q load and its gradient inside the dQ kernel's epilogue (prefill_fwd_rope):
# only the shared k head goes through the RoPE kernel.  False rotates every head first, as the
# reference does (outputs bitwise equal; dq_rope within one bf16 rounding).
ROPE_FOLD = True

# submodules whose weights a decode step reads (their version counters key the recorded step)
_STEP_WEIGHT_MODULES = ("q_down", "qk_rope", "kv_down", "q_up", "k_up", "v_up", "o_proj")

# With autograd off, bf16 weights and input, a one-token step with a cache replays a HIP graph
# of the whole step (DecodeGraph bound to the cache's own buffers), recorded on first use and
# again when the buffers grow, the batch changes or a weight changes; False keeps the eager
# kernels.  Outputs equal the eager path's whenever both split the context alike (always for
# caches of 1024 positions or more at B = 32).
AUTO_GRAPH = True
_AUTO_GRAPH_MIN_STEPS = 16  # replays per recording below which a module stops recording


# With autograd off, a chunk of T > 1 tokens over a cache with one shared k_rope head runs the
# reference's absorbed form (transformer.py:249-291) on prefill_cached, reading the cache in its
# latent form, whenever the per-key cost model below favours it over up-projecting the cache
# into per-head K and V for prefill_fwd; False always up-projects.
ABSORBED_PREFILL = True
# multiply-adds per key and head: absorbed T (2 DL + 64) against expanded DL (dn + dv) +
# T (dn + dr + dv); the absorbed kernel is taken when its count times this factor (the ratio of
# the two paths' measured throughputs) is the smaller
_ABSORBED_COST = 1.3

_SPLIT_ALIGN = 256  # hipBLASLt tiles N in multiples of this well


def _split_pays(M: int, N: int) -> bool:
    """Whether x [M, K] @ W[N, K]^T runs as two products (see _linear_split_cols): large M, and N
    past a multiple of 256 by a remainder."""
    return M >= 1024 and N > _SPLIT_ALIGN and N % _SPLIT_ALIGN != 0


def _linear_split_cols(x, W):
    """``x @ W^T`` (no bias, autograd off) as two hipBLASLt products writing the columns of one
    output: the first N - N % 256 columns, then the rest.  At the benchmark down-projections
    (ModelArgs.mla_baseline dims: M = 24576 rows, K = 2048) one product of N = 2624 took 275 us and the 2560 + 64 pair 197 us,
    since hipBLASLt tiles N = 2560 well and 2624 poorly.  Results equal the one product to
    within its rounding (the two use different kernels)."""
    N = W.size(0)
    main = N - N % _SPLIT_ALIGN
    x2 = x.reshape(-1, x.size(-1))
    y = torch.empty(x2.size(0), N, dtype=W.dtype, device=x.device)
    torch.mm(x2, W[:main].t(), out=y[:, :main])
    torch.mm(x2, W[main:].t(), out=y[:, main:])
    return y.view(*x.shape[:-1], N)


class _SplitColsLinear(torch.autograd.Function):
    """``x @ W^T`` with the forward as _linear_split_cols and the backward as single products
    (the split does not pay there: dx 214 against 243 us, dW 336 against 397 us at the benchmark
    down-projections)."""

    @staticmethod
    def forward(ctx, x, W):
        ctx.save_for_backward(x, W)
        return _linear_split_cols(x, W)

    @staticmethod
    def backward(ctx, dy):
        x, W = ctx.saved_tensors
        dy2 = dy.reshape(-1, dy.size(-1))
        dx = (dy2 @ W).view(x.shape) if ctx.needs_input_grad[0] else None
        dW = dy2.t() @ x.reshape(-1, x.size(-1)) if ctx.needs_input_grad[1] else None
        return dx, dW


class RotaryEmbedding(nn.Module):
    """bf16 cos/sin tables ``[max_seq_len, dim/2]`` (transformer.py:29-53).

    The tables are built exactly as the reference builds them (fp32 angles, cos/sin
    in fp32, stored as bf16) because they are part of the numerics the kernels and
    the reference share; ``forward`` returns the first ``seq_len`` rows in x's dtype.
    """

    def __init__(self, dim, max_seq_len=8192, theta=10000.0):
        super().__init__()
        freqs = 1.0 / (theta ** (torch.arange(0, dim, 2).float() / dim))
        t = torch.arange(max_seq_len)
        freqs = torch.outer(t, freqs).float()
        self.register_buffer("cos_cached", freqs.cos().to(torch.bfloat16), persistent=False)
        self.register_buffer("sin_cached", freqs.sin().to(torch.bfloat16), persistent=False)

    def forward(self, x, seq_len):
        cos = self.cos_cached[:seq_len]
        sin = self.sin_cached[:seq_len]
        if cos.dtype != x.dtype:
            cos = cos.to(dtype=x.dtype)
            sin = sin.to(dtype=x.dtype)
        return cos, sin


def apply_rope(x, cos, sin):
    """Split-half RoPE of ``x [..., T, 64]`` with ``cos/sin [T, 32]`` on the GPU
    (transformer.py:55-60).  The tables must hold bf16 values (as RotaryEmbedding's do)."""
    if x.size(-1) != 64 or cos.shape[-2:] != (x.size(-2), 32):
        raise ValueError("apply_rope: x must be [..., T, 64] with cos/sin [T, 32]")
    lead = x.shape[:-2]
    x4 = x.reshape(-1, 1, x.size(-2), 64).transpose(1, 2)  # [N, T, 1, 64] view
    c = cos.to(torch.bfloat16).contiguous()
    s = sin.to(torch.bfloat16).contiguous()
    y = ops.rope(x4, c, s, 0, False)
    return y.transpose(1, 2).reshape(*lead, x.size(-2), 64)


class MLA(nn.Module):
    """DeepSeek-style MLA with decoupled RoPE (transformer.py:128-316) on MI355X kernels."""

    def __init__(self, args):
        super().__init__()
        H, dn, dr, dv, hr = mla_dims(args)
        if dr != 64:
            raise ValueError("MLA: the decoupled RoPE slice is fixed at 64 (transformer.py:138)")
        self.n_heads = H
        self.head_dim = int(args.head_dim)
        self.d_model = int(args.d_model)
        self.rope_dim = dr
        self.content_dim = dn
        self.v_head_dim = dv
        self.n_k_rope_heads = hr
        self.d_latent = int(args.d_latent)
        q_lora = int(getattr(args, "q_lora_rank", self.d_latent))

        self.q_down = nn.Linear(self.d_model, q_lora, bias=False)
        self.q_up = nn.Linear(q_lora, H * dn, bias=False)
        self.qk_rope = nn.Linear(self.d_model, (H + hr) * dr, bias=False)
        self.kv_down = nn.Linear(self.d_model, self.d_latent, bias=False)
        self.k_up = nn.Linear(self.d_latent, H * dn, bias=False)
        self.v_up = nn.Linear(self.d_latent, H * dv, bias=False)
        self.o_proj = nn.Linear(H * dv, self.d_model, bias=False)
        max_seq_len = int(getattr(args, "max_seq_len", 8192))
        self.rope = RotaryEmbedding(dr, max_seq_len=max_seq_len, theta=float(getattr(args, "rope_theta", 10000.0)))
        # transformer.py:170 and SDPA's default: 1/sqrt(q/k head dim)
        self.scale = 1.0 / math.sqrt(dn + dr)
        self._old_rope_keys = ("q_rope.weight", "k_rope.weight")

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                              error_msgs):
        # legacy checkpoints hold separate q_rope/k_rope weights: fuse them (transformer.py:177-200)
        qk_key, q_key, k_key = prefix + "qk_rope.weight", prefix + "q_rope.weight", prefix + "k_rope.weight"
        if qk_key not in state_dict and q_key in state_dict and k_key in state_dict:
            state_dict[qk_key] = torch.cat([state_dict[q_key], state_dict[k_key]], dim=0)
            state_dict.pop(q_key, None)
            state_dict.pop(k_key, None)
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                                      error_msgs)

    def _cached_weight(self, name, make, dtype):
        """A derived weight (``make()``, cast to ``dtype``) kept while the parameters it reads
        are unchanged (same storage and version counter); autograd off only."""
        params = [self.q_down.weight, self.qk_rope.weight, self.kv_down.weight] if name == "down" else \
            [getattr(self, name.split(":")[0]).weight]
        key = tuple((w.data_ptr(), w._version) for w in params) + (dtype,)
        cache = self.__dict__.setdefault("_derived", {})
        hit = cache.get(name)
        if hit is None or hit[0] != key:
            with torch.no_grad():
                hit = (key, make().to(dtype).contiguous())
            cache[name] = hit
        return hit[1]

    def _auto_graph_ok(self, x):
        """The one-token cached step may replay a recorded graph: autograd off; with autocast off,
        bf16 weights and a bf16 input; under bf16 autocast, bf16 or fp32 weights and a bf16 or fp32
        input (fp32 weights under bf16 autocast is how the reference's generation loop runs,
        CLI.py:294); not inside a graph capture or torch.compile, and the module has not given up
        recording.  The recording keeps its cache in bf16, which is the reference's cache dtype in
        those cases; an fp32 module outside autocast takes the eager kernels, whose cache stays
        fp32 as the reference's does (transformer.py:215-218, :241-244)."""
        if not AUTO_GRAPH or torch.is_grad_enabled():
            return False
        wdt, amp = self._step_weights()[-1].dtype, torch.is_autocast_enabled("cuda")
        if amp:
            ok = autocast_bf16() and wdt in (torch.bfloat16, torch.float32) and x.dtype in (torch.bfloat16,
                                                                                            torch.float32)
        else:
            ok = wdt == torch.bfloat16 and x.dtype == wdt
        return (ok and not self.__dict__.get("_graph_off", False) and not torch.compiler.is_compiling()
                and not torch.cuda.is_current_stream_capturing())

    def _step_graph(self, store, L0, B):
        """The recorded step bound to ``store``'s buffers, recorded again when the buffers
        (a grown or a different store), the batch, a weight or the RoPE table changed.  One
        recording is kept; it holds the buffers it writes until it is replaced or released.
        A module whose recordings serve fewer than _AUTO_GRAPH_MIN_STEPS steps each (caches
        used in turn) goes back to the eager kernels: None is returned from then on."""
        key = (id(store), store.latent.data_ptr(), store.capacity, B, self.rope.cos_cached.data_ptr(),
               autocast_bf16()) + tuple((w.data_ptr(), w._version) for w in self._step_weights())
        st = self.__dict__.setdefault("_graph_state", {"key": None, "graph": None, "records": 0, "steps": 0})
        if st["key"] != key:
            st["graph"] = st["key"] = None  # release the old recording and its buffers first
            st["records"] += 1
            if st["records"] > 4 and st["records"] * _AUTO_GRAPH_MIN_STEPS > st["steps"]:
                self.__dict__["_graph_off"] = True
                self.release_decode_graph()
                return None
            cache = {"latent": store.latent[:, :L0], "k_rope": store.k_rope[:, :, :L0], "seq_len": L0}
            graph = DecodeGraph(self, cache, buffers=(store.latent, store.k_rope))
            graph.mla = None  # replays need only the recording; no module -> state -> module cycle
            st["graph"], st["key"] = graph, key
        st["steps"] += 1
        return st["graph"]

    def _step_weights(self):
        """The weights a decode step reads (q_down, qk_rope, kv_down, q_up, k_up, v_up, o_proj), taken
        from the submodules' parameter dicts: the per-token step reads them on every call, and
        ``nn.Module.__getattr__`` costs more host time than the dict lookups (a weight that is not a
        plain parameter, e.g. a parametrization's, is read as an attribute)."""
        mods, out = self._modules, []
        for name in _STEP_WEIGHT_MODULES:
            mod = mods[name]
            w = mod._parameters.get("weight")
            out.append(w if w is not None else mod.weight)
        return out

    def release_decode_graph(self):
        """Drop the recorded decode step (and the cache buffers it holds)."""
        self.__dict__.pop("_graph_state", None)

    def refresh_weights(self):
        """Forget every weight-derived copy: the bf16 / transposed copies of the few-row products,
        the concatenated down-projection weight and the recorded decode step.  They are rebuilt
        from the parameters on next use.  The module notices ordinary parameter updates by their
        storage and version counter; an update that bypasses the version counter (``p.data.copy_``,
        a kernel writing through ``p.data_ptr()``, such as a fused optimizer) must be followed by
        this call before the next inference step."""
        self.__dict__.pop("_derived", None)
        self.__dict__.pop("_down_w", None)
        self.__dict__.pop("_down_key", None)
        self.release_decode_graph()


    def _absorbed_prefill_ok(self, T, k_pos):
        """Whether a T-token chunk over a cache takes the absorbed kernel: autograd off, one
        shared k_rope head, a built d_latent, and fewer multiply-adds per key (weighted by
        _ABSORBED_COST) than up-projecting every cached row into per-head K and V."""
        if not ABSORBED_PREFILL or torch.is_grad_enabled() or k_pos.size(1) != 1 \
                or self.d_latent not in kernels.PREFILL_CACHED_LATENT:
            return False
        DL, dn, dr, dv = self.d_latent, self.content_dim, self.rope_dim, self.v_head_dim
        return _ABSORBED_COST * T * (2 * DL + dr) < DL * (dn + dv) + T * (dn + dr + dv)

    def _rows_dims_ok(self):
        """Whether every product of the decode step fits linear_rows' shape limits (K a
        multiple of 128 up to ROWS_MAX_K, N a multiple of 4)."""
        H, dn, dv = self.n_heads, self.content_dim, self.v_head_dim
        n_down = self.q_down.weight.size(0) + self.qk_rope.weight.size(0) + self.kv_down.weight.size(0)
        return all(kernels.rows_fit(K, N) for K, N in (
            (self.d_model, n_down), (self.q_up.weight.size(1), H * dn), (dn, self.d_latent), (H * dv, self.d_model)))

    def _rows_path(self, x):
        """Few-row bf16 products (the decode step): autograd off, at most ROWS_FAST_M rows, and
        bf16 arithmetic (bf16 weights, or bf16 autocast)."""
        if torch.is_grad_enabled() or x.size(0) * x.size(1) > kernels.ROWS_FAST_M or not self._rows_dims_ok():
            return False
        if torch.is_autocast_enabled("cuda"):
            return torch.get_autocast_dtype("cuda") == torch.bfloat16
        return self.o_proj.weight.dtype == torch.bfloat16

    def _down_proj(self, x):
        """``q_down(x)``, ``qk_rope(x)`` and ``kv_down(x)`` (transformer.py:208-213) as one GEMM
        over the concatenated weights ``[q_lora + (H + Hr) 64 + d_latent, d_model]``: x is read
        once instead of three times.  The outputs are column views of the one result.  With
        autograd off the concatenation (in the autocast dtype) is kept while the three
        weights are unchanged.  For many rows and N past a multiple of 256 (2624 at the
        ModelArgs.mla_baseline dims) the forward product runs as two (_linear_split_cols)."""
        ws = (self.q_down.weight, self.qk_rope.weight, self.kv_down.weight)
        sizes = [w.size(0) for w in ws]
        split = _split_pays(x.numel() // x.size(-1), sum(sizes)) and not torch.compiler.is_compiling()
        if torch.is_grad_enabled() and any(w.requires_grad for w in ws):
            W = torch.cat(ws, 0)
            if split:  # autocast's casts, made explicit for the autograd Function
                dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else W.dtype
                return _SplitColsLinear.apply(x.to(dt), W.to(dt)).split(sizes, dim=-1)
        else:
            dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else ws[0].dtype
            key = tuple((w.data_ptr(), w._version) for w in ws) + (dt,)
            if getattr(self, "_down_key", None) != key:
                self._down_w = torch.cat([w.detach() for w in ws], 0).to(dt)
                self._down_key = key
            W = self._down_w
        if not split or W.requires_grad:
            return torch.nn.functional.linear(x, W).split(sizes, dim=-1)
        if torch.is_grad_enabled() and x.requires_grad:  # frozen weights, the input's gradient
            return _SplitColsLinear.apply(x.to(W.dtype), W).split(sizes, dim=-1)
        return _linear_split_cols(x.to(W.dtype), W).split(sizes, dim=-1)

    @staticmethod
    def _bf16(t):
        return t if t.dtype == torch.bfloat16 else t.to(torch.bfloat16)

    def forward(self, x, kv_cache=None, use_cache=False):
        if not x.is_cuda:
            raise RuntimeError("transformer_amd.MLA runs on a ROCm GPU only (no CPU path)")
        B, T, _ = x.shape
        H, dn, dr, dv, hr = self.n_heads, self.content_dim, self.rope_dim, self.v_head_dim, self.n_k_rope_heads
        pos_offset = int(kv_cache["seq_len"]) if kv_cache is not None else 0  # :205
        kv_len = pos_offset + T
        n_pos = self._modules["rope"]._buffers["cos_cached"].size(0)  # RoPE table rows
        if kv_len > n_pos:
            raise ValueError(f"MLA: position {kv_len} exceeds the RoPE table ({n_pos} rows); raise max_seq_len")

        if T == 1 and use_cache and ROPE_APPEND and self._auto_graph_ok(x):
            # the whole one-token step replayed from a recording bound to the cache's buffers
            store, L0 = latent_cache.reserve(kv_cache, B, 1, hr, self.d_latent, dr, torch.bfloat16, x.device, n_pos)
            graph = self._step_graph(store, L0, B)
            if graph is not None:
                y = graph.step_at(x, L0).clone()
                return y, latent_cache.commit(store, L0 + 1)[2]
            kv_cache = latent_cache.commit(store, L0)[2]  # the eager step below appends to the same store
        rows = self._rows_path(x)
        if rows:
            # the decode step's few-row products (:208-213 as one, then q_up) on linear_rows
            bf = torch.bfloat16
            Wd = self._cached_weight("down", lambda: torch.cat(
                [self.q_down.weight, self.qk_rope.weight, self.kv_down.weight], 0), bf)
            sizes = [self.q_down.weight.size(0), self.qk_rope.weight.size(0), self.kv_down.weight.size(0)]
            q_low, qk_pos, kv_new = ops.linear_rows(x.reshape(B * T, -1).to(bf), Wd).view(B, T, -1).split(sizes, -1)
            Wq = self._cached_weight("q_up", lambda: self.q_up.weight, bf)
            if ROPE_APPEND and use_cache:
                # q_up (:208) beside the RoPE with the cache append (:215-218, :228-244), which read
                # only the down-projections: one launch, bit for bit the two kernels
                store, L0 = latent_cache.reserve(kv_cache, B, T, hr, self.d_latent, dr, bf, x.device, n_pos)
                q_content, q_rope = ops.linear_rows_rope_append(
                    q_low.reshape(B * T, -1), Wq, qk_pos.view(B, T, H + hr, dr), kv_new, store.latent, store.k_rope,
                    self.rope.cos_cached, self.rope.sin_cached, None, None, L0, H, None)
                appended = latent_cache.commit(store, L0 + T)
                return self._forward_cached(x, q_content.view(B, T, H, dn), q_rope, None, kv_new, kv_cache, pos_offset,
                                            q_content.dtype, appended, rows)
            q_content = ops.linear_rows(q_low.reshape(B * T, -1), Wq).view(B, T, -1)  # :208
        else:
            q_low, qk_pos, kv_new = self._down_proj(x)  # :208-213, one GEMM (see _down_proj)
            q_content = self.q_up(q_low)  # [B,T,H*dn]                   :208
        cdt = q_content.dtype

        q_nope = q_content.view(B, T, H, dn)
        qk4 = qk_pos.view(B, T, H + hr, dr)
        if ROPE_APPEND and use_cache and not torch.is_grad_enabled() and qk4.dtype == torch.bfloat16 \
                and kv_new.dtype == torch.bfloat16:
            # RoPE with the cache append (:215-218, :228-244) in one kernel: the rotated k heads
            # and the new latent rows go straight into the preallocated store's slots
            store, L0 = latent_cache.reserve(kv_cache, B, T, hr, self.d_latent, dr, torch.bfloat16, x.device,
                                             self.rope.cos_cached.size(0))
            q_rope = ops.rope_append(qk4, kv_new, store.latent, store.k_rope, self.rope.cos_cached,
                                     self.rope.sin_cached, None, None, L0, H, None)
            appended = latent_cache.commit(store, L0 + T)
            return self._forward_cached(x, q_nope, q_rope, None, kv_new, kv_cache, pos_offset, cdt, appended, rows)

        cos, sin = self.rope.cos_cached, self.rope.sin_cached
        if ROPE_FOLD and not use_cache and qk4.dtype == torch.bfloat16:
            # training / no-cache branch: the q heads' rotation (:228-233) happens in the attention
            # kernel's Q load (and its gradient in the dQ epilogue); only the k heads go through
            # the RoPE kernel here (:236-239)
            k_rope_new = ops.rope(qk4[:, :, H:], cos, sin, pos_offset, False)  # [B,T,Hr,64]
            q_rope = None
        else:
            # one kernel rotates the q heads and the k heads (:228-239)
            roped = ops.rope(qk4, cos, sin, pos_offset, False)
            q_rope = roped[:, :, :H]
            k_rope_new = roped[:, :, H:]  # [B,T,Hr,64]

        if use_cache:
            return self._forward_cached(x, q_nope, q_rope, k_rope_new, kv_new, kv_cache, pos_offset, cdt, None, rows)

        # training / no-cache branch (:306-316).  SDPA's is_causal is top-left aligned, so a
        # cache passed with use_cache=False keeps q_offset = 0 as in the reference.
        if kv_cache is not None:
            kv_latent = torch.cat([kv_cache["latent"].to(kv_new.dtype), kv_new], dim=1)
            k_rope = torch.cat([kv_cache["k_rope"].to(k_rope_new.dtype), k_rope_new.transpose(1, 2)], dim=2)
            k_rope = k_rope.transpose(1, 2)
        else:
            kv_latent, k_rope = kv_new, k_rope_new
        k_nope = self.k_up(kv_latent).view(B, kv_len, H, dn)
        v = self.v_up(kv_latent).view(B, kv_len, H, dv)
        b = self._bf16
        if q_rope is None:
            o, _, _ = ops.prefill_fwd_rope(b(q_nope), qk4[:, :, :H], b(k_nope), b(k_rope), b(v), cos, sin, self.scale,
                                           True, 0, pos_offset, torch.is_grad_enabled())
        else:
            o, _ = ops.prefill_fwd(b(q_nope), b(q_rope), b(k_nope), b(k_rope), b(v), self.scale, True, 0)
        out = o.reshape(B, T, H * dv).to(cdt)
        return self.o_proj(out), None

    def _forward_cached(self, x, q_nope, q_rope, k_rope_new, kv_new, kv_cache, pos_offset, cdt, appended=None,
                        rows=False):
        B, T = x.shape[:2]
        H, dn, dv = self.n_heads, self.content_dim, self.v_head_dim
        new_cache = None
        if appended is not None:  # rope_append already wrote the new positions
            kv_latent, k_pos, new_cache = appended
        elif not torch.is_grad_enabled():
            # append in place to preallocated buffers (:215-218, :241-244 without the O(L) copy)
            kv_latent, k_pos, new_cache = latent_cache.append(kv_cache, kv_new, k_rope_new.transpose(1, 2),
                                                              self.rope.cos_cached.size(0))
        elif kv_cache is not None:
            kv_latent = torch.cat([kv_cache["latent"].to(kv_new.dtype), kv_new], dim=1)  # :215-218
            k_pos = torch.cat([kv_cache["k_rope"].to(k_rope_new.dtype), k_rope_new.transpose(1, 2)], dim=2)  # :241
        else:
            kv_latent = kv_new
            k_pos = k_rope_new.transpose(1, 2).contiguous()  # [B,Hr,T,64]
        kv_len = kv_latent.size(1)
        b = self._bf16
        if T == 1:
            # absorbed decode (:249-291): q_lat = q_nope W_UK, ctx = softmax(s) c_kv, out = ctx W_UV^T
            if rows:
                # W_UK transposed per head [H, DL, dn], so the absorption is H few-row products
                Wkt = self._cached_weight("k_up:t", lambda: self.k_up.weight.view(H, dn, self.d_latent).transpose(1, 2),
                                          torch.bfloat16)
                q_lat = ops.linear_rows(b(q_nope.reshape(B, H, dn)), Wkt).view(B, H, self.d_latent)
            else:
                Wk = b(self.k_up.weight).view(H, dn, self.d_latent)
                q_lat = ops.absorb_q(b(q_nope.reshape(B, H, dn)), Wk)  # [B,H,DL]
            # the W_UV product (:290-291) runs inside the decode's split merge and writes the
            # [B, H * dv] rows o_proj reads
            Wv = b(self.v_up.weight).view(H, dv, self.d_latent)
            out, _ = ops.decode_out(q_lat, b(q_rope.reshape(B, H, -1)), b(kv_latent), b(k_pos), None, Wv,
                                    self.scale, 0)
            out = out.reshape(B, 1, H * dv).to(cdt)
        elif self._absorbed_prefill_ok(T, k_pos):
            # T > 1 in the absorbed form (:249-291) with the bottom-right mask of :273-281: q_lat =
            # q_nope W_UK and ctx W_UV^T as per-head batched products, the attention over the cache's
            # latent rows on prefill_cached (query t at position pos_offset + t)
            DL = self.d_latent
            Wk = self._cached_weight("k_up", lambda: self.k_up.weight.view(H, dn, DL), torch.bfloat16)
            qn = b(q_nope).permute(2, 0, 1, 3).reshape(H, B * T, dn)
            q_lat = torch.bmm(qn, Wk).view(H, B, T, DL).permute(1, 2, 0, 3)  # [B,T,H,DL] view
            ctx, _ = ops.prefill_cached(q_lat, b(q_rope), b(kv_latent), b(k_pos), pos_offset, self.scale, True)
            Wvt = self._cached_weight("v_up:t", lambda: self.v_up.weight.view(H, dv, DL).transpose(1, 2),
                                      torch.bfloat16)  # [H, DL, dv]
            out = torch.bmm(ctx.permute(2, 0, 1, 3).reshape(H, B * T, DL), Wvt)  # [H, B*T, dv]
            out = out.view(H, B, T, dv).permute(1, 2, 0, 3).reshape(B, T, H * dv).to(cdt)
        else:
            # T > 1 with the bottom-right causal mask of :273-281 (q_offset = pos_offset)
            k_nope = self.k_up(kv_latent).view(B, kv_len, H, dn)
            v = self.v_up(kv_latent).view(B, kv_len, H, dv)
            o, _ = ops.prefill_fwd(b(q_nope), b(q_rope), b(k_nope), b(k_pos.transpose(1, 2)), b(v), self.scale,
                                   True, pos_offset)
            out = o.reshape(B, T, H * dv).to(cdt)
        if new_cache is None:
            new_cache = {"latent": kv_latent.detach(), "k_rope": k_pos.detach(), "seq_len": kv_len}  # :295-299
        if rows:
            Wo = self._cached_weight("o_proj", lambda: self.o_proj.weight, torch.bfloat16)
            return ops.linear_rows(b(out).reshape(B * T, -1), Wo).view(B, T, -1).to(cdt), new_cache  # :300
        return self.o_proj(out), new_cache


def release_decode_graphs(model: torch.nn.Module, refresh_weights: bool = False) -> int:
    """Release the recorded decode step of every MLA module in ``model`` (with the cache buffers
    each recording holds), e.g. when a generation ends; with ``refresh_weights`` also drop their
    weight-derived copies (after updating weights in a way that bypasses the version counter).
    Returns the number of MLA modules visited."""
    n = 0
    for mod in model.modules():
        if isinstance(mod, MLA):
            if refresh_weights:
                mod.refresh_weights()
            else:
                mod.release_decode_graph()
            n += 1
    return n
