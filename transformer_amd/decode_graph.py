"""One MLA decode step (one token per sequence) captured in a HIP graph.

In eager mode a decode step of the module launches about a dozen kernels (the
down-projections as one GEMM, ``q_up``, RoPE, the cache append, the W_UK absorption, the
decode and its merge with the W_UV product, ``o_proj``) for a few tens of microseconds of
GPU work, so launch overhead dominates.  Here RoPE, both cache appends, the new
sequence lengths and the next position are one kernel (``rope_append``) that reads the
position on the device; the position alternates between two buffers, so the step is
recorded twice (even and odd steps) and the recordings are replayed in turn.  ``DecodeGraph`` keeps every value that changes from step to step on the
device: the write position, and with it the RoPE table row and the sequence lengths the
decode kernel reads.  The whole step is then recorded once and replayed per token:

    y, cache = mla(prompt, None, True)          # prefill (eager)
    step = DecodeGraph(mla, cache)             # copies the cache into fixed buffers, records
    for x in tokens:                           # x: [B, 1, d_model]
        y = step(x)                            # replays; y is valid until the next call
    cache = step.cache()                       # the reference's cache dict at the current length

It computes what ``mla(x, cache, True)`` computes for one token (transformer.py:202-300
with T == 1), with the cache append at transformer.py:215-218,241-244 done in place.
Per-sequence lengths let the decode kernel split each sequence's own length over its
workgroups, so the capacity-sized cache costs no idle work.

The module's weights are read when the graph is recorded: W_UK and W_UV are taken as
the bf16 copies the decode needs at that point, and the three down-projection weights as
one concatenated copy this object owns, so a ``DecodeGraph`` is for inference with fixed
weights (make a new one after changing them).  The projections run in the module's own
dtype (bf16 or fp32), or in bf16 for fp32 weights when bf16 autocast is on at construction
(what the eager module computes there; the reference's generation loop runs that way,
CLI.py:294), from bf16 copies held here; RoPE, the cache and the attention are bf16, as in
the eager module.  All sequences of the batch
advance together, as in the reference's cache (one ``seq_len`` per dict).
"""
from __future__ import annotations

import torch

from . import kernels  # registers the ops; ROWS_FAST_M

ops = kernels.eager  # torch.ops.mla_mi355x, without the dispatcher where nothing needs it


def _record(graph: torch.cuda.CUDAGraph, dev: torch.device, body):
    """Record ``body()`` into ``graph`` on a side stream; returns what ``body`` returns.

    A recording registers torch's CUDA RNG, whose graph state (two tensors) is made by the
    first recording that finds none.  Made under inference mode, those would be inference
    tensors that no later recording outside inference mode can update (it then fails and
    leaves the generator mid-capture).  So the recording begins with inference mode off; if the
    state already exists as inference tensors (made by a recording elsewhere), it begins as
    before, under the caller's mode, which also completes the generator's capture cycle."""
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        begun = False
        if torch.is_inference_mode_enabled():
            try:
                with torch.inference_mode(False):
                    graph.capture_begin()
                begun = True
            except RuntimeError:
                pass
        if not begun:
            graph.capture_begin()
        try:
            out = body()
        finally:
            graph.capture_end()
    torch.cuda.current_stream(dev).wait_stream(side)
    return out


def autocast_bf16() -> bool:
    """Whether bf16 autocast is on for the GPU."""
    return torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16


class DecodeGraph:
    def __init__(self, mla, cache: dict, capacity: int | None = None, *, buffers=None):
        """``buffers``: bf16 ``(latent [B, C, d_latent], k_rope [B, Hr, C, 64])`` whose first
        ``seq_len`` positions already hold the cache; the graph then appends into them in place
        (capacity C) instead of into copies of its own."""
        lat, kr = cache["latent"], cache["k_rope"]
        if not lat.is_cuda:
            raise RuntimeError("DecodeGraph: the cache must be on the GPU")
        L0 = int(cache["seq_len"])
        B, _, DL = lat.shape
        Hr = kr.size(1)
        rows = mla.rope.cos_cached.size(0)
        if buffers is not None:
            C = buffers[0].size(1)
        else:
            C = rows if capacity is None else int(capacity)
        if not (L0 < C <= rows):
            raise ValueError(f"DecodeGraph: capacity {C} must exceed the cache length {L0} and fit the "
                             f"RoPE table ({rows} rows)")
        self.mla = mla
        self.capacity = C
        wdt = mla.o_proj.weight.dtype
        # the step's arithmetic: the weights' dtype, or bf16 for fp32 weights under bf16 autocast
        cdt = torch.bfloat16 if wdt == torch.float32 and autocast_bf16() else wdt
        self.dtype = cdt
        dev = lat.device
        H, dn, dv = mla.n_heads, mla.content_dim, mla.v_head_dim
        if buffers is not None:
            self.latent, self.k_rope = buffers
            if (self.latent.dtype != torch.bfloat16 or self.k_rope.dtype != torch.bfloat16
                    or tuple(self.latent.shape) != (B, C, DL) or tuple(self.k_rope.shape) != (B, Hr, C, kr.size(3))):
                raise ValueError("DecodeGraph: buffers must be bf16 [B, C, d_latent] and [B, Hr, C, 64]")
        else:
            self.latent = torch.zeros(B, C, DL, dtype=torch.bfloat16, device=dev)
            self.k_rope = torch.zeros(B, Hr, C, kr.size(3), dtype=torch.bfloat16, device=dev)
            self.latent[:, :L0].copy_(lat)
            self.k_rope[:, :, :L0].copy_(kr)
        # the position of the next token alternates between two device buffers: the step that
        # reads one writes the next position into the other, so no step increments in place
        self.pos = [torch.full((1,), L0, dtype=torch.int64, device=dev),
                    torch.full((1,), L0 + 1, dtype=torch.int64, device=dev)]
        self.seq_lens = torch.full((B,), L0 + 1, dtype=torch.int32, device=dev)  # written by every step
        self.n = L0  # the same count on the host (the device counter is advanced by the replay)
        self.x = torch.zeros(B, 1, mla.d_model, dtype=cdt, device=dev)
        # bf16 absorption weights: W_UK [H, dn, DL] and W_UV [H, dv, DL] (transformer.py:252-254,290-291)
        self.w_uk = mla.k_up.weight.detach().view(H, dn, DL).to(torch.bfloat16).contiguous()
        self.w_uv = mla.v_up.weight.detach().view(H, dv, DL).to(torch.bfloat16).contiguous()
        # q_down, qk_rope and kv_down as one product over a concatenated weight held here, so the
        # recorded graph reads memory this object keeps alive (:208-213)
        downs = (mla.q_down.weight, mla.qk_rope.weight, mla.kv_down.weight)
        self.w_down = torch.cat([w.detach() for w in downs], 0).to(cdt).contiguous()
        self.down_sizes = [w.size(0) for w in downs]
        # q_up and o_proj in the step's dtype (the module's own tensors when that is theirs)
        self.w_qup = mla.q_up.weight.detach().to(cdt).contiguous()
        self.w_o = mla.o_proj.weight.detach().to(cdt).contiguous()
        # bf16 arithmetic runs the step's few-row products on linear_rows: the down-projections,
        # q_up, W_UK transposed per head [H, DL, dn] (the absorption as H products) and o_proj
        # (the module's own choice for this batch: autograd off, bf16, at most ROWS_FAST_M rows and
        # every product within the kernel's shape limits)
        self.rows = cdt == torch.bfloat16 and mla._rows_dims_ok() and B <= kernels.ROWS_FAST_M
        if self.rows:
            self.w_ukt = self.w_uk.transpose(1, 2).contiguous()

        # warm up on a side stream (library handles and allocator pools), then record; the
        # warm-up step writes the slot at L0 and advances pos, so both are restored
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(2):
                self._body(self.pos[0], self.pos[1])
                self.pos[0].fill_(L0)
        torch.cuda.current_stream(dev).wait_stream(side)
        # two recordings: even steps read pos[0] and write pos[1], odd steps the reverse
        self.graphs, self.ys = [], []
        for i in range(2):
            graph = torch.cuda.CUDAGraph()
            with torch.no_grad():
                self.ys.append(_record(graph, dev, lambda: self._body(self.pos[i], self.pos[1 - i])))
            self.graphs.append(graph)
        self.L0 = L0
        self.next_rec = 0  # recording i reads pos[i] and writes pos[1 - i]

    def _body(self, pos, pos_next):
        m = self.mla
        x = self.x
        B = x.size(0)
        H, dn, dr, dv, hr = m.n_heads, m.content_dim, m.rope_dim, m.v_head_dim, m.n_k_rope_heads
        # RoPE at the device-side position, with the append at pos (:215-218, :228-244) and the new
        # lengths in the same kernel; the cache is bf16 (a no-op cast for a bf16 module)
        bf = torch.bfloat16
        cos, sin = m.rope.cos_cached, m.rope.sin_cached
        if self.rows:
            q_low, qk_pos, kv_new = ops.linear_rows(x.view(B, -1), self.w_down).split(self.down_sizes, -1)  # :208-213
            # q_up (:208) and the RoPE + append read only the down-projections: one launch
            q_content, q_rope = ops.linear_rows_rope_append(q_low, self.w_qup, qk_pos.view(B, 1, H + hr, dr),
                                                            kv_new.view(B, 1, -1), self.latent, self.k_rope, cos,
                                                            sin, pos, self.seq_lens, 0, H, pos_next)
        else:
            q_low, qk_pos, kv_new = torch.nn.functional.linear(x, self.w_down).split(self.down_sizes, -1)
            q_content = torch.nn.functional.linear(q_low, self.w_qup)
            q_rope = ops.rope_append(qk_pos.view(B, 1, H + hr, dr).to(bf), kv_new.view(B, 1, -1).to(bf), self.latent,
                                     self.k_rope, cos, sin, pos, self.seq_lens, 0, H, pos_next)
        seq_lens = self.seq_lens
        # absorbed decode (:249-291)
        if self.rows:
            q_lat = ops.linear_rows(q_content.view(B, H, dn), self.w_ukt)  # [B,H,DL] (:252-254)
        else:
            q_lat = ops.absorb_q(q_content.view(B, H, dn).to(torch.bfloat16), self.w_uk)
        out, _ = ops.decode_out(q_lat, q_rope.reshape(B, H, dr).to(torch.bfloat16), self.latent, self.k_rope,
                                seq_lens, self.w_uv, m.scale, 0)  # W_UV (:290-291) in the split merge
        if self.rows:
            return ops.linear_rows(out.view(B, H * dv), self.w_o).view(B, 1, -1)  # :300
        out = out.reshape(B, 1, H * dv).to(x.dtype)
        return torch.nn.functional.linear(out, self.w_o)  # :300

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        """One decode step for ``x [B, 1, d_model]``; returns the layer output ``[B, 1, d_model]``
        (a buffer the next call overwrites).  ``x`` is copied into the recording's input buffer
        ``self.x`` (one small copy kernel); a caller that writes its input there directly, e.g. as
        the output of the op before, passes ``self.x`` and the copy is skipped."""
        return self.step_at(x, self.n)

    def step_at(self, x: torch.Tensor, pos: int) -> torch.Tensor:
        """The decode step of ``x`` written at position ``pos`` (the cache holds positions
        [0, pos)); the next position on the device is reset when ``pos`` is not the one the
        previous step left there."""
        if tuple(x.shape) != tuple(self.x.shape):
            raise ValueError(f"DecodeGraph: x must be {tuple(self.x.shape)}, got {tuple(x.shape)}")
        if not 0 <= pos < self.capacity:
            raise ValueError(f"DecodeGraph: position {pos} outside the cache's {self.capacity} positions")
        i = self.next_rec
        if pos != self.n:
            self.pos[i].fill_(pos)
        if x.data_ptr() != self.x.data_ptr():  # an input written into ``self.x`` needs no copy
            self.x.copy_(x)
        self.graphs[i].replay()
        self.next_rec = 1 - i
        self.n = pos + 1
        return self.ys[i]

    def cache(self) -> dict:
        """The cache in the reference's dict format (views of this object's buffers)."""
        return {"latent": self.latent[:, :self.n], "k_rope": self.k_rope[:, :, :self.n], "seq_len": self.n}
