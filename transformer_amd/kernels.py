"""torch operators over the C ABI (``torch.ops.mla_mi355x.*``).

Each op validates its tensors, allocates outputs with torch on the input's
device, and enqueues the HIP kernel on torch's current stream through the
C-ABI library.  Ops are registered with ``torch.library.custom_op`` (fake
kernels for tracing, autograd formulas for RoPE and prefill), so the MLA module
works under autocast, activation checkpointing and ``torch.compile``.  ``eager``
(at the end) runs the same bodies without the dispatcher for eager callers.

There is no CPU path: a CPU tensor, or a missing library, raises.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _lib
from ._lib import DecodeArgs, PrefillBwdArgs, PrefillFwdArgs, RopeArgs, Strides

ROPE_DIM = 64
SUPPORTED_NOPE = (64, 128)
SUPPORTED_V = (128,)
SUPPORTED_LATENT = (64, 128, 256, 384, 512)
# prefill_bwd: form dQ from the dS blocks the dK/dV pass stores (the workspace then holds
# 2 KiB per 32 x 32 block, up to 8 GiB), or set False to recompute S and dP in the dQ pass
BWD_STORED_DS = True


# ----------------------------------------------------------------- helpers

# the op bodies by name, as registered: ``eager`` below calls them without the dispatcher
_BODIES = {}


def _op(name: str, mutates_args=()):
    """Register ``fn`` as ``torch.ops.mla_mi355x.<name>`` and keep its body for ``eager``."""
    def register(fn):
        _BODIES[name] = fn
        return torch.library.custom_op(f"mla_mi355x::{name}", mutates_args=mutates_args)(fn)
    return register


def _require_gpu(op: str, *tensors: Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{op}: tensors must be on a ROCm GPU (got {t.device}); "
                               "transformer_amd has no CPU implementation")


def _stream(t: Tensor) -> int:
    """torch's current stream on ``t``'s device, as the raw ``hipStream_t`` handle (the same
    value as ``torch.cuda.current_stream(t.device).cuda_stream``, without building a Stream)."""
    return torch._C._cuda_getCurrentRawStream(t.get_device())


def _aligned4(t: Tensor, vec_elems: int) -> Tensor:
    """Return ``t`` (or a contiguous copy) with unit innermost stride, 16-byte aligned
    base and strides that are multiples of ``vec_elems`` elements."""
    ok = (t.stride(-1) == 1 or t.size(-1) == 1) and t.data_ptr() % 16 == 0 and all(
        s % vec_elems == 0 for s, n in zip(t.stride()[:-1], t.shape[:-1]) if n > 1)
    return t if ok else t.contiguous()


def _st4(t: Tensor, zero_head: bool = False) -> Strides:
    """Strides (b, t, h) of a [B, T, heads, dim] tensor; size-1 dims get stride 0."""
    sb = t.stride(0) if t.size(0) > 1 else 0
    stt = t.stride(1) if t.size(1) > 1 else 0
    sh = 0 if (zero_head or t.size(2) == 1) else t.stride(2)
    return Strides(sb, stt, sh)


def _ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _bf16(op: str, **tensors: Tensor) -> None:
    for name, t in tensors.items():
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{op}: {name} must be bfloat16, got {t.dtype}")


# ----------------------------------------------------------------- RoPE

def _rope_launch(x: Tensor, y: Tensor, cos: Tensor, sin: Tensor, pos_offset: int, inverse: bool) -> None:
    args = RopeArgs(
        x=x.data_ptr(), y=y.data_ptr(), cos=cos.data_ptr(), sin=sin.data_ptr(),
        B=x.size(0), T=x.size(1), n_heads=x.size(2), table_rows=cos.size(0), pos_offset=int(pos_offset),
        x_stride=Strides(x.stride(0), x.stride(1), x.stride(2)),
        y_stride=Strides(y.stride(0), y.stride(1), y.stride(2)),
        dtype=_lib.MLA_DTYPE_BF16 if x.dtype == torch.bfloat16 else _lib.MLA_DTYPE_F32,
        inverse=1 if inverse else 0)
    _lib.check(_lib.entry("mla_rope")(ctypes.byref(args), _stream(x)), "mla_rope")


def _rope_check(x: Tensor, cos: Tensor, sin: Tensor) -> None:
    _require_gpu("mla_mi355x::rope", x, cos, sin)
    if x.dim() != 4 or x.size(-1) != ROPE_DIM:
        raise ValueError(f"rope: x must be [B, T, heads, {ROPE_DIM}], got {tuple(x.shape)}")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"rope: x must be bf16 or fp32, got {x.dtype}")
    if cos.dtype != torch.bfloat16 or sin.dtype != torch.bfloat16 or cos.shape != sin.shape \
            or cos.dim() != 2 or cos.size(1) != ROPE_DIM // 2 or not cos.is_contiguous() or not sin.is_contiguous():
        raise ValueError("rope: cos/sin must be contiguous bf16 [rows, 32] tables")


@_op("rope", mutates_args=())
def rope(x: Tensor, cos: Tensor, sin: Tensor, pos_offset: int, inverse: bool = False) -> Tensor:
    """Decoupled RoPE of ``x [B, T, heads, 64]`` at positions ``pos_offset + t``
    (transformer.py:55-60 over the q and k heads at once); returns a new tensor."""
    _rope_check(x, cos, sin)
    x = _aligned4(x, 8 if x.dtype == torch.bfloat16 else 4)
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if y.numel():
        _rope_launch(x, y, cos, sin, pos_offset, inverse)
    return y


@rope.register_fake
def _(x, cos, sin, pos_offset, inverse=False):
    return torch.empty(x.shape, dtype=x.dtype, device=x.device)


def _rope_setup(ctx, inputs, output):
    _, cos, sin, pos_offset, inverse = inputs
    ctx.save_for_backward(cos, sin)
    ctx.pos_offset = pos_offset
    ctx.inverse = inverse


def _rope_backward(ctx, grad):
    cos, sin = ctx.saved_tensors
    # R is orthogonal: the gradient is the rotation by the opposite angle
    return torch.ops.mla_mi355x.rope(grad, cos, sin, ctx.pos_offset, not ctx.inverse), None, None, None, None


rope.register_autograd(_rope_backward, setup_context=_rope_setup)


@_op("rope_", mutates_args=("x",))
def rope_(x: Tensor, cos: Tensor, sin: Tensor, pos_offset: int, inverse: bool = False) -> None:
    """In-place variant of :func:`rope` (no autograd); ``x`` must already satisfy the
    kernel's alignment (unit innermost stride, 16-byte aligned rows)."""
    _rope_check(x, cos, sin)
    if _aligned4(x, 8 if x.dtype == torch.bfloat16 else 4) is not x:
        raise ValueError("rope_: x is not 16-byte aligned with unit innermost stride")
    if x.numel():
        _rope_launch(x, x, cos, sin, pos_offset, inverse)


@rope_.register_fake
def _(x, cos, sin, pos_offset, inverse=False):
    return None


def _rope_append_args(op, qk, c_new, latent, k_cache, cos, sin, pos, seq_lens, pos_offset, n_q_heads, pos_next):
    """Checks of :func:`rope_append` and its argument struct: ``(args, q_out, keep)``, ``keep`` holding
    any re-laid-out inputs alive until the launch is enqueued."""
    _require_gpu(op, qk, c_new, latent, k_cache, cos, sin, pos, seq_lens)
    _bf16(op, qk=qk, c_new=c_new, latent=latent, k_cache=k_cache, cos=cos, sin=sin)
    if qk.dim() != 4 or qk.size(-1) != ROPE_DIM or c_new.dim() != 3 or latent.dim() != 3 or k_cache.dim() != 4:
        raise ValueError(f"{op}: expected qk [B,T,H+Hr,64], c_new [B,T,DL], latent [B,C,DL], k_cache [B,Hr,C,64]")
    B, T, NH, _ = qk.shape
    H = int(n_q_heads)
    Hr = NH - H
    DL = c_new.size(-1)
    C = latent.size(1)
    if not 0 < H < NH or tuple(c_new.shape[:2]) != (B, T) or latent.size(0) != B or latent.size(2) != DL \
            or tuple(k_cache.shape) != (B, Hr, C, ROPE_DIM) or cos.shape != sin.shape or cos.size(-1) != 32:
        raise ValueError(f"{op}: inconsistent shapes qk {tuple(qk.shape)} (H={H}) c_new {tuple(c_new.shape)} "
                         f"latent {tuple(latent.shape)} k_cache {tuple(k_cache.shape)}")
    for name, t in (("pos", pos), ("pos_next", pos_next)):
        if t is not None and (t.dtype != torch.int64 or t.numel() != 1):
            raise ValueError(f"{op}: {name} must be one int64 element on the device")
    if pos_next is not None and pos is not None and pos_next.data_ptr() == pos.data_ptr():
        raise ValueError(f"{op}: pos_next must be a different buffer from pos")
    if seq_lens is not None and (seq_lens.dtype != torch.int32 or tuple(seq_lens.shape) != (B,)
                                 or not seq_lens.is_contiguous()):
        raise ValueError(f"{op}: seq_lens must be a contiguous int32 [B]")
    for name, t in (("latent", latent), ("k_cache", k_cache)):
        if t.stride(-1) != 1 or t.data_ptr() % 16 or any(x % 8 for x in t.stride()[:-1]):
            raise ValueError(f"{op}: {name} must have a unit inner stride, 16-byte alignment and strides "
                             "that are multiples of 8 (it is written in place)")
    qk = _aligned4(qk, 8)
    c_new = _aligned4(c_new, 8)
    cos = cos.contiguous()
    sin = sin.contiguous()
    q_out = torch.empty(B, T, H, ROPE_DIM, dtype=torch.bfloat16, device=qk.device)
    sb = lambda t, i: t.stride(i) if t.size(i) > 1 else 0
    args = _lib.RopeAppendArgs(
        qk=qk.data_ptr(), q_out=q_out.data_ptr(), c_new=c_new.data_ptr(), latent=latent.data_ptr(),
        k_cache=k_cache.data_ptr(), cos=cos.data_ptr(), sin=sin.data_ptr(), pos_dev=_ptr(pos),
        seq_lens=_ptr(seq_lens), pos_next=_ptr(pos_next), B=B, T=T, H=H, Hr=Hr, d_latent=DL, capacity=C,
        table_rows=cos.size(0),
        pos_offset=int(pos_offset), qk_stride=Strides(sb(qk, 0), sb(qk, 1), qk.stride(2)),
        q_stride=_st4(q_out), c_new_sb=sb(c_new, 0), c_new_st=sb(c_new, 1), latent_sb=sb(latent, 0),
        latent_st=latent.stride(1), k_cache_sb=sb(k_cache, 0), k_cache_sh=sb(k_cache, 1),
        k_cache_st=k_cache.stride(2))
    return args, q_out, (qk, c_new, cos, sin)


@_op("rope_append", mutates_args=("latent", "k_cache", "seq_lens", "pos_next"))
def rope_append(qk: Tensor, c_new: Tensor, latent: Tensor, k_cache: Tensor, cos: Tensor, sin: Tensor,
                pos: Optional[Tensor], seq_lens: Optional[Tensor], pos_offset: int, n_q_heads: int,
                pos_next: Optional[Tensor]) -> Tensor:
    """RoPE of the new tokens with the cache append in one kernel (transformer.py:215-244):
    ``qk [B, T, H + Hr, 64]`` (the rope slice of the qk_rope GEMM: q heads, then k heads),
    ``c_new [B, T, DL]`` (kv_down output), caches ``latent [B, C, DL]`` and
    ``k_cache [B, Hr, C, 64]``.  The k heads are rotated into ``k_cache[:, :, p]`` and
    ``c_new`` is copied to ``latent[:, p]`` for ``p = pos_offset + pos + t`` (``pos``: an
    optional int64 device scalar, read by the kernel); ``seq_lens`` (int32 [B], optional)
    receives the new length, and ``pos_next`` (an int64 device scalar other than ``pos``,
    optional) the next position.  Returns the rotated q heads ``[B, T, H, 64]``."""
    op = "mla_mi355x::rope_append"
    args, q_out, keep = _rope_append_args(op, qk, c_new, latent, k_cache, cos, sin, pos, seq_lens, pos_offset,
                                          n_q_heads, pos_next)
    _lib.check(_lib.entry("mla_rope_append")(ctypes.byref(args), _stream(q_out)), op)
    return q_out


@rope_append.register_fake
def _(qk, c_new, latent, k_cache, cos, sin, pos, seq_lens, pos_offset, n_q_heads, pos_next):
    B, T = qk.shape[:2]
    return qk.new_empty(B, T, int(n_q_heads), ROPE_DIM)


# ----------------------------------------------------------------- prefill

def _prefill_check(op, q_nope, q_rope, k_nope, k_rope, v):
    _require_gpu(op, q_nope, q_rope, k_nope, k_rope, v)
    _bf16(op, q_nope=q_nope, q_rope=q_rope, k_nope=k_nope, k_rope=k_rope, v=v)
    for name, t in (("q_nope", q_nope), ("q_rope", q_rope), ("k_nope", k_nope), ("k_rope", k_rope), ("v", v)):
        if t.dim() != 4:
            raise ValueError(f"{op}: {name} must be [B, T, heads, dim], got {tuple(t.shape)}")
    B, Tq, H, dn = q_nope.shape
    Tk = k_nope.size(1)
    Hr = k_rope.size(2)
    if dn not in SUPPORTED_NOPE or v.size(-1) not in SUPPORTED_V:
        raise ValueError(f"{op}: head dims nope={dn}, v={v.size(-1)} not built (nope {SUPPORTED_NOPE}, v {SUPPORTED_V})")
    if tuple(q_rope.shape) != (B, Tq, H, ROPE_DIM) or tuple(k_nope.shape) != (B, Tk, H, dn) \
            or tuple(k_rope.shape) != (B, Tk, Hr, ROPE_DIM) or Hr not in (1, H) \
            or tuple(v.shape[:3]) != (B, Tk, H):
        raise ValueError(f"{op}: inconsistent shapes q_nope {tuple(q_nope.shape)} q_rope {tuple(q_rope.shape)} "
                         f"k_nope {tuple(k_nope.shape)} k_rope {tuple(k_rope.shape)} v {tuple(v.shape)}")
    return B, Tq, Tk, H, Hr, dn, v.size(-1)


def _rope_tables_check(op, cos, sin, rows_needed):
    if cos.dtype != torch.bfloat16 or sin.dtype != torch.bfloat16 or cos.shape != sin.shape or cos.dim() != 2 \
            or cos.size(1) != ROPE_DIM // 2 or not cos.is_contiguous() or not sin.is_contiguous():
        raise ValueError(f"{op}: cos/sin must be contiguous bf16 [rows, 32] tables")
    if rows_needed > cos.size(0):
        raise ValueError(f"{op}: positions up to {rows_needed - 1} exceed the RoPE table ({cos.size(0)} rows)")


def _prefill_fwd_impl(op, q_nope, q_rope, k_nope, k_rope, v, scale, causal, q_offset, cos=None, sin=None,
                      q_pos_offset=0, save_rotated=False):
    B, Tq, Tk, H, Hr, dn, dv = _prefill_check(op, q_nope, q_rope, k_nope, k_rope, v)
    q_nope, q_rope, k_nope, k_rope, v = (_aligned4(t, 8) for t in (q_nope, q_rope, k_nope, k_rope, v))
    o = torch.empty(B, Tq, H, dv, dtype=torch.bfloat16, device=q_nope.device)
    lse = torch.empty(B, H, Tq, dtype=torch.float32, device=q_nope.device)
    q_rot = torch.empty(B, Tq, H, ROPE_DIM, dtype=torch.bfloat16, device=q_nope.device) if save_rotated \
        else q_nope.new_empty(0)
    if o.numel() == 0:
        return o, lse, q_rot
    args = PrefillFwdArgs(
        q_nope=q_nope.data_ptr(), q_rope=q_rope.data_ptr(), k_nope=k_nope.data_ptr(), k_rope=k_rope.data_ptr(),
        v=v.data_ptr(), o=o.data_ptr(), lse=lse.data_ptr(),
        B=B, H=H, Tq=Tq, Tk=Tk, d_nope=dn, d_rope=ROPE_DIM, d_v=dv,
        q_nope_stride=_st4(q_nope), q_rope_stride=_st4(q_rope), k_nope_stride=_st4(k_nope),
        k_rope_stride=_st4(k_rope, zero_head=(Hr == 1)), v_stride=_st4(v), o_stride=_st4(o),
        scale=float(scale), causal=1 if causal else 0, q_offset=int(q_offset), workspace=None, workspace_bytes=0,
        rope_cos=None, rope_sin=None, rope_rows=0, q_pos_offset=0, q_rope_out=None)
    if cos is not None:
        _require_gpu(op, cos, sin)
        _rope_tables_check(op, cos, sin, int(q_pos_offset) + Tq)
        args.rope_cos, args.rope_sin, args.rope_rows = cos.data_ptr(), sin.data_ptr(), cos.size(0)
        args.q_pos_offset = int(q_pos_offset)
        if save_rotated:
            args.q_rope_out, args.q_rope_out_stride = q_rot.data_ptr(), _st4(q_rot)
    nbytes = int(_lib.entry("mla_prefill_fwd_workspace_bytes")(ctypes.byref(args)))
    if nbytes:  # small grids: key-split partials (the call runs unsplit without them)
        ws = _alloc_workspace(nbytes, o.device)
        args.workspace = ws.data_ptr()
        args.workspace_bytes = nbytes
    _lib.check(_lib.entry("mla_prefill_fwd")(ctypes.byref(args), _stream(o)), op)
    return o, lse, q_rot


@_op("prefill_fwd", mutates_args=())
def prefill_fwd(q_nope: Tensor, q_rope: Tensor, k_nope: Tensor, k_rope: Tensor, v: Tensor,
                scale: float, causal: bool = True, q_offset: int = 0) -> Tuple[Tensor, Tensor]:
    """Flash attention over nope/rope-split Q and K (no concat materialised).

    Returns ``o [B, Tq, H, d_v]`` bf16 and ``lse [B, H, Tq]`` fp32 (natural log).
    Restates transformer.py:311-314 (q_offset 0) and the masked absorbed prefill
    (transformer.py:273-291, q_offset = pos_offset)."""
    o, lse, _ = _prefill_fwd_impl("mla_mi355x::prefill_fwd", q_nope, q_rope, k_nope, k_rope, v, scale, causal,
                                  q_offset)
    return o, lse


@_op("prefill_fwd_rope", mutates_args=())
def prefill_fwd_rope(q_nope: Tensor, q_rope: Tensor, k_nope: Tensor, k_rope: Tensor, v: Tensor, cos: Tensor,
                     sin: Tensor, scale: float, causal: bool = True, q_offset: int = 0, q_pos_offset: int = 0,
                     save_rotated: bool = True) -> Tuple[Tensor, Tensor, Tensor]:
    """:func:`prefill_fwd` with the queries' RoPE (transformer.py:228-233) folded into the kernel's
    Q load: ``q_rope`` is the unrotated slice (the qk_rope projection's q heads, :209-210), row t
    is rotated at position ``q_pos_offset + t`` with the bf16 tables ``cos``/``sin``, bit for bit
    as :func:`rope`.  Returns ``(o, lse, q_rope_rotated)``; the rotated slice (what the backward
    needs) is written only with ``save_rotated`` (else an empty tensor).  Its backward rotates
    dq_rope back inside the dQ kernel's epilogue.  ``k_rope`` is already rotated."""
    return _prefill_fwd_impl("mla_mi355x::prefill_fwd_rope", q_nope, q_rope, k_nope, k_rope, v, scale, causal,
                             q_offset, cos, sin, q_pos_offset, save_rotated)


@prefill_fwd_rope.register_fake
def _(q_nope, q_rope, k_nope, k_rope, v, cos, sin, scale, causal=True, q_offset=0, q_pos_offset=0,
      save_rotated=True):
    B, Tq, H, _ = q_nope.shape
    return (q_nope.new_empty(B, Tq, H, v.size(-1)), q_nope.new_empty(B, H, Tq, dtype=torch.float32),
            q_nope.new_empty(B, Tq, H, ROPE_DIM) if save_rotated else q_nope.new_empty(0))


@prefill_fwd.register_fake
def _(q_nope, q_rope, k_nope, k_rope, v, scale, causal=True, q_offset=0):
    B, Tq, H, _ = q_nope.shape
    return (q_nope.new_empty(B, Tq, H, v.size(-1)), q_nope.new_empty(B, H, Tq, dtype=torch.float32))


@_op("prefill_bwd", mutates_args=())
def prefill_bwd(dout: Tensor, q_nope: Tensor, q_rope: Tensor, k_nope: Tensor, k_rope: Tensor, v: Tensor,
                o: Tensor, lse: Tensor, scale: float, causal: bool = True, q_offset: int = 0,
                cos: Optional[Tensor] = None, sin: Optional[Tensor] = None, q_pos_offset: int = 0
                ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Gradients (dq_nope, dq_rope, dk_nope, dk_rope, dv) of :func:`prefill_fwd`
    (the SDPA backward of transformer.py:314).  A shared k_rope head receives the sum
    over query heads.  With ``cos``/``sin`` (the backward of :func:`prefill_fwd_rope`),
    ``q_rope`` is the rotated slice and dq_rope is returned for the unrotated one, rotated
    back at positions ``q_pos_offset + t`` in the dQ kernel before its rounding."""
    op = "mla_mi355x::prefill_bwd"
    B, Tq, Tk, H, Hr, dn, dv = _prefill_check(op, q_nope, q_rope, k_nope, k_rope, v)
    _require_gpu(op, dout, o, lse)
    _bf16(op, dout=dout, o=o)
    if tuple(dout.shape) != (B, Tq, H, dv) or tuple(o.shape) != (B, Tq, H, dv) or tuple(lse.shape) != (B, H, Tq) \
            or lse.dtype != torch.float32:
        raise ValueError(f"{op}: dout/o must be [B, Tq, H, d_v] bf16 and lse [B, H, Tq] fp32")
    dout, q_nope, q_rope, k_nope, k_rope, v, o = (_aligned4(t, 8) for t in (dout, q_nope, q_rope, k_nope, k_rope, v, o))
    lse = lse.contiguous()
    dev = q_nope.device
    dq_nope = torch.empty(B, Tq, H, dn, dtype=torch.bfloat16, device=dev)
    dq_rope = torch.empty(B, Tq, H, ROPE_DIM, dtype=torch.bfloat16, device=dev)
    dk_nope = torch.empty(B, Tk, H, dn, dtype=torch.bfloat16, device=dev)
    dk_rope = torch.empty(B, Tk, Hr, ROPE_DIM, dtype=torch.bfloat16, device=dev)
    dvv = torch.empty(B, Tk, H, dv, dtype=torch.bfloat16, device=dev)
    if dq_nope.numel() == 0 and dk_nope.numel() == 0:
        return dq_nope, dq_rope, dk_nope, dk_rope, dvv
    args = PrefillBwdArgs(
        dout=dout.data_ptr(), q_nope=q_nope.data_ptr(), q_rope=q_rope.data_ptr(), k_nope=k_nope.data_ptr(),
        k_rope=k_rope.data_ptr(), v=v.data_ptr(), o=o.data_ptr(), lse=lse.data_ptr(),
        dq_nope=dq_nope.data_ptr(), dq_rope=dq_rope.data_ptr(), dk_nope=dk_nope.data_ptr(),
        dk_rope=dk_rope.data_ptr(), dv=dvv.data_ptr(), workspace=None, workspace_bytes=0,
        B=B, H=H, Tq=Tq, Tk=Tk, d_nope=dn, d_rope=ROPE_DIM, d_v=dv,
        dout_stride=_st4(dout), q_nope_stride=_st4(q_nope), q_rope_stride=_st4(q_rope),
        k_nope_stride=_st4(k_nope), k_rope_stride=_st4(k_rope, zero_head=(Hr == 1)), v_stride=_st4(v),
        o_stride=_st4(o), dq_nope_stride=_st4(dq_nope), dq_rope_stride=_st4(dq_rope),
        dk_nope_stride=_st4(dk_nope), dk_rope_stride=_st4(dk_rope, zero_head=(Hr == 1)), dv_stride=_st4(dvv),
        scale=float(scale), causal=1 if causal else 0, q_offset=int(q_offset),
        rope_cos=None, rope_sin=None, rope_rows=0, q_pos_offset=0)
    if cos is not None:
        _require_gpu(op, cos, sin)
        _rope_tables_check(op, cos, sin, int(q_pos_offset) + Tq)
        args.rope_cos, args.rope_sin, args.rope_rows = cos.data_ptr(), sin.data_ptr(), cos.size(0)
        args.q_pos_offset = int(q_pos_offset)
    ws, nbytes = _bwd_workspace(args, dev)
    args.workspace = ws.data_ptr()
    args.workspace_bytes = nbytes
    _lib.check(_lib.entry("mla_prefill_bwd")(ctypes.byref(args), _stream(dq_nope)), op)
    return dq_nope, dq_rope, dk_nope, dk_rope, dvv


def _bwd_workspace(args: PrefillBwdArgs, dev: torch.device) -> Tuple[Tensor, int]:
    """The backward's workspace: room for the stored dS blocks when BWD_STORED_DS, else (or when
    that allocation fails for lack of memory) the smaller workspace of the recompute path,
    which gives the same gradients."""
    if BWD_STORED_DS:
        nbytes = int(_lib.entry("mla_prefill_bwd_workspace_bytes")(ctypes.byref(args)))
        try:
            return _alloc_workspace(nbytes, dev), nbytes
        except torch.OutOfMemoryError:
            pass
    nbytes = int(_lib.entry("mla_prefill_bwd_workspace_min_bytes")(ctypes.byref(args)))
    return _alloc_workspace(nbytes, dev), nbytes


def _alloc_workspace(nbytes: int, dev: torch.device) -> Tensor:
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)


@prefill_bwd.register_fake
def _(dout, q_nope, q_rope, k_nope, k_rope, v, o, lse, scale, causal=True, q_offset=0, cos=None, sin=None,
      q_pos_offset=0):
    return (torch.empty_like(q_nope, memory_format=torch.contiguous_format),
            torch.empty_like(q_rope, memory_format=torch.contiguous_format),
            torch.empty_like(k_nope, memory_format=torch.contiguous_format),
            torch.empty_like(k_rope, memory_format=torch.contiguous_format),
            torch.empty_like(v, memory_format=torch.contiguous_format))


def _prefill_setup(ctx, inputs, output):
    q_nope, q_rope, k_nope, k_rope, v, scale, causal, q_offset = inputs
    o, lse = output
    ctx.save_for_backward(q_nope, q_rope, k_nope, k_rope, v, o, lse)
    ctx.scale, ctx.causal, ctx.q_offset = scale, causal, q_offset
    ctx.mark_non_differentiable(lse)


def _prefill_backward(ctx, do, dlse):
    q_nope, q_rope, k_nope, k_rope, v, o, lse = ctx.saved_tensors
    grads = torch.ops.mla_mi355x.prefill_bwd(do, q_nope, q_rope, k_nope, k_rope, v, o, lse,
                                             ctx.scale, ctx.causal, ctx.q_offset)
    return (*grads, None, None, None)


prefill_fwd.register_autograd(_prefill_backward, setup_context=_prefill_setup)


def _prefill_rope_setup(ctx, inputs, output):
    q_nope, q_rope, k_nope, k_rope, v, cos, sin, scale, causal, q_offset, q_pos_offset, save_rotated = inputs
    o, lse, q_rot = output
    ctx.save_for_backward(q_nope, q_rot, k_nope, k_rope, v, o, lse, cos, sin)
    ctx.scale, ctx.causal, ctx.q_offset, ctx.q_pos_offset = scale, causal, q_offset, q_pos_offset
    ctx.saved_rotated = save_rotated
    ctx.mark_non_differentiable(lse, q_rot)


def _prefill_rope_backward(ctx, do, dlse, dqrot):
    if not ctx.saved_rotated:
        raise RuntimeError("prefill_fwd_rope: the backward needs save_rotated=True in the forward")
    q_nope, q_rot, k_nope, k_rope, v, o, lse, cos, sin = ctx.saved_tensors
    grads = torch.ops.mla_mi355x.prefill_bwd(do, q_nope, q_rot, k_nope, k_rope, v, o, lse, ctx.scale, ctx.causal,
                                             ctx.q_offset, cos, sin, ctx.q_pos_offset)
    return (*grads, None, None, None, None, None, None, None)


prefill_fwd_rope.register_autograd(_prefill_rope_backward, setup_context=_prefill_rope_setup)


# ----------------------------------------------------------------- decode

def _decode_args(op, q_lat, q_rope, c_kv, k_rope, seq_lens, scale, num_splits, ctx, lse):
    """Validated DecodeArgs (and the possibly re-laid-out inputs, which must outlive the launch)."""
    _require_gpu(op, q_lat, q_rope, c_kv, k_rope, seq_lens)
    _bf16(op, q_lat=q_lat, q_rope=q_rope, c_kv=c_kv, k_rope=k_rope)
    if q_lat.dim() != 3 or q_rope.dim() != 3 or c_kv.dim() != 3 or k_rope.dim() != 4:
        raise ValueError(f"{op}: expected q_lat [B,H,DL], q_rope [B,H,64], c_kv [B,L,DL], k_rope [B,Hr,L,64]")
    B, H, DL = q_lat.shape
    L = c_kv.size(1)
    Hr = k_rope.size(1)
    if DL not in SUPPORTED_LATENT:
        raise ValueError(f"{op}: d_latent {DL} not built (supported {SUPPORTED_LATENT})")
    if tuple(q_rope.shape) != (B, H, ROPE_DIM) or tuple(c_kv.shape) != (B, L, DL) \
            or tuple(k_rope.shape) != (B, Hr, L, ROPE_DIM) or Hr not in (1, H):
        raise ValueError(f"{op}: inconsistent shapes q_lat {tuple(q_lat.shape)} q_rope {tuple(q_rope.shape)} "
                         f"c_kv {tuple(c_kv.shape)} k_rope {tuple(k_rope.shape)}")
    if seq_lens is not None:
        if seq_lens.dtype != torch.int32 or tuple(seq_lens.shape) != (B,):
            raise ValueError(f"{op}: seq_lens must be int32 [B]")
        seq_lens = seq_lens.contiguous()

    def fix(t):
        ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(
            s % 8 == 0 for s, n in zip(t.stride()[:-1], t.shape[:-1]) if n > 1)
        return t if ok else t.contiguous()

    q_lat, q_rope, c_kv, k_rope = fix(q_lat), fix(q_rope), fix(c_kv), fix(k_rope)
    sb = lambda t, i: t.stride(i) if t.size(i) > 1 else 0
    args = DecodeArgs(
        q_lat=q_lat.data_ptr(), q_rope=q_rope.data_ptr(), c_kv=c_kv.data_ptr(), k_rope=k_rope.data_ptr(),
        seq_lens=_ptr(seq_lens), ctx=_ptr(ctx), lse=lse.data_ptr(), workspace=None, workspace_bytes=0,
        B=B, H=H, L=L, d_latent=DL, d_rope=ROPE_DIM, n_k_rope_heads=Hr,
        q_lat_sb=sb(q_lat, 0), q_lat_sh=sb(q_lat, 1), q_rope_sb=sb(q_rope, 0), q_rope_sh=sb(q_rope, 1),
        c_kv_sb=sb(c_kv, 0), c_kv_st=sb(c_kv, 1),
        k_rope_sb=sb(k_rope, 0), k_rope_sh=0 if Hr == 1 else k_rope.stride(1), k_rope_st=sb(k_rope, 2),
        ctx_sb=ctx.stride(0) if ctx is not None else 0, ctx_sh=ctx.stride(1) if ctx is not None else 0,
        scale=float(scale), num_splits=int(num_splits))
    return args, (q_lat, q_rope, c_kv, k_rope, seq_lens)


@_op("decode", mutates_args=())
def decode(q_lat: Tensor, q_rope: Tensor, c_kv: Tensor, k_rope: Tensor, seq_lens: Optional[Tensor],
           scale: float, num_splits: int = 0) -> Tuple[Tensor, Tensor]:
    """Absorbed latent decode (transformer.py:249-286 for T == 1).

    ``q_lat [B, H, DL]``, ``q_rope [B, H, 64]``, ``c_kv [B, L, DL]``,
    ``k_rope [B, Hr, L, 64]`` (Hr in {1, H}), optional int32 ``seq_lens [B]``.
    Returns ``ctx [B, H, DL]`` bf16 (= softmax(s) c_kv) and ``lse [B, H]`` fp32."""
    op = "mla_mi355x::decode"
    B, H, DL = q_lat.shape
    dev = q_lat.device
    ctx = torch.empty(B, H, DL, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, H, dtype=torch.float32, device=dev)
    # `keep` holds any re-laid-out copies of the inputs alive until the launch is enqueued
    args, keep = _decode_args(op, q_lat, q_rope, c_kv, k_rope, seq_lens, scale, num_splits, ctx, lse)
    if ctx.numel() == 0:
        return ctx, lse
    nbytes = int(_lib.entry("mla_decode_workspace_bytes")(ctypes.byref(args)))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    args.workspace = ws.data_ptr()
    args.workspace_bytes = nbytes
    _lib.check(_lib.entry("mla_decode")(ctypes.byref(args), _stream(ctx)), op)
    return ctx, lse


@decode.register_fake
def _(q_lat, q_rope, c_kv, k_rope, seq_lens, scale, num_splits=0):
    B, H, DL = q_lat.shape
    return q_lat.new_empty(B, H, DL), q_lat.new_empty(B, H, dtype=torch.float32)


@_op("absorb_q", mutates_args=())
def absorb_q(q_nope: Tensor, w_uk: Tensor) -> Tensor:
    """``q_lat[b, h] = q_nope[b, h] W_UK[h]`` (transformer.py:252-254) for the decode step:
    ``q_nope [B, H, d_nope]`` (any strides with a unit inner stride, e.g. ``q_up``'s output
    viewed per head), ``w_uk [H, d_nope, DL]`` bf16 (``k_up.weight.view(H, d_nope, DL)``).
    Returns ``q_lat [B, H, DL]`` bf16 (fp32 accumulation)."""
    op = "mla_mi355x::absorb_q"
    _require_gpu(op, q_nope, w_uk)
    _bf16(op, q_nope=q_nope, w_uk=w_uk)
    if q_nope.dim() != 3 or w_uk.dim() != 3 or w_uk.size(0) != q_nope.size(1) or w_uk.size(1) != q_nope.size(2):
        raise ValueError(f"{op}: expected q_nope [B, H, dn] and w_uk [H, dn, DL]; got {tuple(q_nope.shape)}, "
                         f"{tuple(w_uk.shape)}")
    B, H, dn = q_nope.shape
    DL = w_uk.size(2)
    if dn not in SUPPORTED_NOPE or DL % 8 or DL > 512:
        raise ValueError(f"{op}: d_nope {dn} (built {SUPPORTED_NOPE}) or d_latent {DL} (multiple of 8, <= 512)")
    if q_nope.stride(-1) != 1:
        q_nope = q_nope.contiguous()
    if not (w_uk.stride(-1) == 1 and w_uk.data_ptr() % 16 == 0 and w_uk.stride(0) % 8 == 0 and w_uk.stride(1) % 8 == 0
            and w_uk.stride(1) >= DL):
        w_uk = w_uk.contiguous()
    out = torch.empty(B, H, DL, dtype=torch.bfloat16, device=q_nope.device)
    if out.numel() == 0:
        return out
    sb = lambda t, i: t.stride(i) if t.size(i) > 1 else 0
    args = _lib.AbsorbQArgs(q_nope=q_nope.data_ptr(), w_uk=w_uk.data_ptr(), q_lat=out.data_ptr(), B=B, H=H, d_nope=dn,
                            d_latent=DL, q_sb=sb(q_nope, 0), q_sh=sb(q_nope, 1), w_uk_sh=w_uk.stride(0),
                            w_uk_sd=w_uk.stride(1), out_sb=out.stride(0), out_sh=out.stride(1))
    _lib.check(_lib.entry("mla_absorb_q")(ctypes.byref(args), _stream(out)), op)
    return out


@absorb_q.register_fake
def _(q_nope, w_uk):
    return q_nope.new_empty(q_nope.size(0), q_nope.size(1), w_uk.size(2))


# ----------------------------------------------------------------- prefill with a cache

PREFILL_CACHED_LATENT = (128, 256, 384, 512)


@_op("prefill_cached", mutates_args=())
def prefill_cached(q_lat: Tensor, q_rope: Tensor, c_kv: Tensor, k_rope: Tensor, L0: int,
                   scale: float, heads_first: bool = False, num_splits: int = 0) -> Tuple[Tensor, Tensor]:
    """Absorbed attention of a T-token chunk over a cache (transformer.py:247-286 with T > 1):
    query t sits at position ``L0 + t`` and sees keys ``0 .. L0 + t`` of the cache, which holds
    the chunk's own keys already.  ``q_lat [B, T, H, DL]``, ``q_rope [B, T, H, 64]``,
    ``c_kv [B, L, DL]``, ``k_rope [B, 1, L, 64]`` (shared by the heads), ``L >= L0 + T``.
    Returns ``ctx [B, T, H, DL]`` bf16 (= softmax(s) c_kv) and ``lse [B, H, T]`` fp32.
    ``heads_first`` stores ctx as ``[H, B, T, DL]`` (the returned ``[B, T, H, DL]`` is a
    permuted view of it), the operand layout of the per-head W_UV product.  ``num_splits``: key
    ranges merged by a second kernel (0 chooses; more than one when the batch would not fill
    the chip)."""
    op = "mla_mi355x::prefill_cached"
    _require_gpu(op, q_lat, q_rope, c_kv, k_rope)
    _bf16(op, q_lat=q_lat, q_rope=q_rope, c_kv=c_kv, k_rope=k_rope)
    if q_lat.dim() != 4 or q_rope.dim() != 4 or c_kv.dim() != 3 or k_rope.dim() != 4:
        raise ValueError(f"{op}: expected q_lat [B,T,H,DL], q_rope [B,T,H,64], c_kv [B,L,DL], k_rope [B,1,L,64]")
    B, T, H, DL = q_lat.shape
    L = c_kv.size(1)
    if DL not in PREFILL_CACHED_LATENT:
        raise ValueError(f"{op}: d_latent {DL} not built (supported {PREFILL_CACHED_LATENT})")
    if tuple(q_rope.shape) != (B, T, H, ROPE_DIM) or tuple(c_kv.shape) != (B, L, DL) \
            or tuple(k_rope.shape) != (B, 1, L, ROPE_DIM):
        raise ValueError(f"{op}: inconsistent shapes q_lat {tuple(q_lat.shape)} q_rope {tuple(q_rope.shape)} "
                         f"c_kv {tuple(c_kv.shape)} k_rope {tuple(k_rope.shape)} (k_rope shared by the heads)")
    L0 = int(L0)
    if L0 < 0 or L0 + T > L:
        raise ValueError(f"{op}: the cache holds {L} rows; the chunk needs L0 + T = {L0 + T}")
    dev = q_lat.device
    ctx = _prefill_cached_ctx(q_lat, heads_first)
    lse = torch.empty(B, H, T, dtype=torch.float32, device=dev)
    if ctx.numel() == 0:
        return ctx, lse
    q_lat, q_rope, c_kv, k_rope = (_aligned4(t, 8) for t in (q_lat, q_rope, c_kv, k_rope))
    sb = lambda t, i: t.stride(i) if t.size(i) > 1 else 0
    args = _lib.PrefillCachedArgs(
        q_lat=q_lat.data_ptr(), q_rope=q_rope.data_ptr(), c_kv=c_kv.data_ptr(), k_rope=k_rope.data_ptr(),
        ctx=ctx.data_ptr(), lse=lse.data_ptr(), B=B, T=T, H=H, L=L, L0=L0, d_latent=DL, d_rope=ROPE_DIM,
        q_lat_stride=_st4(q_lat), q_rope_stride=_st4(q_rope), ctx_stride=_st4(ctx),
        c_kv_sb=sb(c_kv, 0), c_kv_st=sb(c_kv, 1), k_rope_sb=sb(k_rope, 0), k_rope_st=sb(k_rope, 2),
        scale=float(scale), num_splits=int(num_splits))
    nbytes = int(_lib.entry("mla_prefill_cached_workspace_bytes")(ctypes.byref(args)))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    args.workspace = ws.data_ptr()
    args.workspace_bytes = nbytes
    _lib.check(_lib.entry("mla_prefill_cached")(ctypes.byref(args), _stream(ctx)), op)
    return ctx, lse


def _prefill_cached_ctx(q_lat: Tensor, heads_first: bool) -> Tensor:
    B, T, H, DL = q_lat.shape
    if heads_first:
        return q_lat.new_empty(H, B, T, DL, dtype=torch.bfloat16).permute(1, 2, 0, 3)
    return q_lat.new_empty(B, T, H, DL, dtype=torch.bfloat16)


@prefill_cached.register_fake
def _(q_lat, q_rope, c_kv, k_rope, L0, scale, heads_first=False, num_splits=0):
    B, T, H, DL = q_lat.shape
    return _prefill_cached_ctx(q_lat, heads_first), q_lat.new_empty(B, H, T, dtype=torch.float32)


@_op("decode_out", mutates_args=())
def decode_out(q_lat: Tensor, q_rope: Tensor, c_kv: Tensor, k_rope: Tensor, seq_lens: Optional[Tensor],
               w_uv: Tensor, scale: float, num_splits: int = 0) -> Tuple[Tensor, Tensor]:
    """Absorbed decode with the per-head W_UV product fused into the split merge
    (transformer.py:249-291 for T == 1): ``out[b, h] = bf16(ctx[b, h]) W_UV[h]^T``.

    ``w_uv [H, d_v, DL]`` bf16 (``v_up.weight.view(H, d_v, DL)``, d_v = 128).  Returns
    ``out [B, H, d_v]`` bf16 (contiguous: the ``[B, H * d_v]`` rows ``o_proj`` reads) and
    ``lse [B, H]`` fp32."""
    op = "mla_mi355x::decode_out"
    B, H, DL = q_lat.shape
    dev = q_lat.device
    _require_gpu(op, w_uv)
    _bf16(op, w_uv=w_uv)
    if w_uv.dim() != 3 or w_uv.size(0) != H or w_uv.size(2) != DL or w_uv.size(1) not in SUPPORTED_V:
        raise ValueError(f"{op}: w_uv must be [H, d_v in {SUPPORTED_V}, DL] = [{H}, 128, {DL}], got {tuple(w_uv.shape)}")
    dv = w_uv.size(1)
    if not (w_uv.stride(-1) == 1 and w_uv.data_ptr() % 16 == 0 and w_uv.stride(0) % 8 == 0
            and w_uv.stride(1) % 8 == 0 and w_uv.stride(1) >= DL):
        w_uv = w_uv.contiguous()
    out = torch.empty(B, H, dv, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, H, dtype=torch.float32, device=dev)
    # `keep` holds any re-laid-out copies of the inputs alive until the launch is enqueued
    dargs, keep = _decode_args(op, q_lat, q_rope, c_kv, k_rope, seq_lens, scale, num_splits, None, lse)
    if out.numel() == 0:
        return out, lse
    args = _lib.DecodeOutArgs(dec=dargs, w_uv=w_uv.data_ptr(), out=out.data_ptr(), w_uv_sh=w_uv.stride(0),
                              w_uv_sd=w_uv.stride(1), out_sb=out.stride(0), out_sh=out.stride(1), d_v=dv)
    nbytes = int(_lib.entry("mla_decode_out_workspace_bytes")(ctypes.byref(args)))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    args.dec.workspace = ws.data_ptr()
    args.dec.workspace_bytes = nbytes
    _lib.check(_lib.entry("mla_decode_out")(ctypes.byref(args), _stream(out)), op)
    return out, lse


@decode_out.register_fake
def _(q_lat, q_rope, c_kv, k_rope, seq_lens, w_uv, scale, num_splits=0):
    B, H, _ = q_lat.shape
    return q_lat.new_empty(B, H, w_uv.size(1)), q_lat.new_empty(B, H, dtype=torch.float32)


# ----------------------------------------------------------------- decode rows

ROWS_FAST_M = 64  # rows up to which linear_rows runs in one pass (the decode step's 32 sequences)
ROWS_MAX_K = 4096  # the kernel stages a workgroup's 16 weight rows whole in LDS


def rows_fit(K: int, N: int) -> bool:
    """Whether a [*, K] x [N, K]^T product fits linear_rows' shape limits."""
    return 0 < K <= ROWS_MAX_K and K % 128 == 0 and N % 4 == 0


def _linear_rows_args(op, x, w):
    """Checks of :func:`linear_rows` and its argument struct: ``(args, y, keep)``, ``keep`` holding
    any re-laid-out inputs alive until the launch is enqueued (an empty y is launched as nothing)."""
    _require_gpu(op, x, w)
    _bf16(op, x=x, w=w)
    grouped = w.dim() == 3
    if grouped:
        if x.dim() != 3 or x.size(1) != w.size(0) or x.size(2) != w.size(2):
            raise ValueError(f"{op}: grouped form needs x [M, G, K] and w [G, N, K]; got {tuple(x.shape)}, "
                             f"{tuple(w.shape)}")
        M, G, K = x.shape
        N = w.size(1)
    else:
        if x.dim() != 2 or w.dim() != 2 or x.size(1) != w.size(1):
            raise ValueError(f"{op}: expected x [M, K] and w [N, K]; got {tuple(x.shape)}, {tuple(w.shape)}")
        M, K = x.shape
        N, G = w.size(0), 1
    if K % 128 or K > ROWS_MAX_K or N % 4:
        raise ValueError(f"{op}: K = {K} must be a multiple of 128 up to {ROWS_MAX_K} and N = {N} of 4")

    def fit(t):
        ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(
            st % 8 == 0 for st, n in zip(t.stride()[:-1], t.shape[:-1]) if n > 1)
        return t if ok else t.contiguous()

    x, w = fit(x), fit(w)
    y = torch.empty((M, G, N) if grouped else (M, N), dtype=torch.bfloat16, device=x.device)
    sb = lambda t, i: t.stride(i) if t.size(i) > 1 else 0
    if grouped:
        args = _lib.LinearRowsArgs(x=x.data_ptr(), w=w.data_ptr(), y=y.data_ptr(), M=M, N=N, K=K, G=G,
                                   x_sm=sb(x, 0), x_sg=sb(x, 1), w_sn=sb(w, 1), w_sg=sb(w, 0),
                                   y_sm=y.stride(0), y_sg=y.stride(1))
    else:
        args = _lib.LinearRowsArgs(x=x.data_ptr(), w=w.data_ptr(), y=y.data_ptr(), M=M, N=N, K=K, G=1,
                                   x_sm=sb(x, 0), x_sg=0, w_sn=sb(w, 0), w_sg=0, y_sm=y.stride(0), y_sg=0)
    return args, y, (x, w)


@_op("linear_rows", mutates_args=())
def linear_rows(x: Tensor, w: Tensor) -> Tensor:
    """``y = x W^T`` for a few rows: ``x [M, K]`` and ``w [N, K]`` give ``y [M, N]``; grouped,
    ``x [M, G, K]`` and ``w [G, N, K]`` give ``y [M, G, N]`` (G products, e.g. one per head).
    bf16, fp32 accumulation.  The decode step's products (transformer.py:208-213, :252-254,
    :300 at T == 1)."""
    op = "mla_mi355x::linear_rows"
    args, y, keep = _linear_rows_args(op, x, w)
    if y.numel() == 0:
        return y
    _lib.check(_lib.entry("mla_linear_rows")(ctypes.byref(args), _stream(y)), op)
    return y


@linear_rows.register_fake
def _(x, w):
    if w.dim() == 3:
        return x.new_empty(x.size(0), w.size(0), w.size(1))
    return x.new_empty(x.size(0), w.size(0))


@_op("linear_rows_rope_append", mutates_args=("latent", "k_cache", "seq_lens", "pos_next"))
def linear_rows_rope_append(x: Tensor, w: Tensor, qk: Tensor, c_new: Tensor, latent: Tensor, k_cache: Tensor,
                            cos: Tensor, sin: Tensor, pos: Optional[Tensor], seq_lens: Optional[Tensor],
                            pos_offset: int, n_q_heads: int, pos_next: Optional[Tensor]) -> Tuple[Tensor, Tensor]:
    """:func:`linear_rows` ``(x, w)`` and :func:`rope_append` in one launch: the decode step's q_up
    product (transformer.py:208) beside the RoPE of the new token with the cache append
    (:215-244).  Returns ``(y, q_rope)``, bit for bit the two ops' results.  ``y`` is a new
    tensor, so it cannot alias the append's buffers; the caller keeps ``x``/``w`` apart from the
    cache it appends to."""
    op = "mla_mi355x::linear_rows_rope_append"
    ra, y, keep_r = _linear_rows_args(op, x, w)
    aa, q_out, keep_a = _rope_append_args(op, qk, c_new, latent, k_cache, cos, sin, pos, seq_lens, pos_offset,
                                          n_q_heads, pos_next)
    if y.numel() == 0:
        ra.M = 0  # nothing to multiply: the launch runs the append only
    _lib.check(_lib.entry("mla_linear_rows_rope_append")(ctypes.byref(ra), ctypes.byref(aa), _stream(q_out)), op)
    return y, q_out


@linear_rows_rope_append.register_fake
def _(x, w, qk, c_new, latent, k_cache, cos, sin, pos, seq_lens, pos_offset, n_q_heads, pos_next):
    B, T = qk.shape[:2]
    y = x.new_empty(x.size(0), w.size(0), w.size(1)) if w.dim() == 3 else x.new_empty(x.size(0), w.size(0))
    return y, qk.new_empty(B, T, int(n_q_heads), ROPE_DIM)


# ----------------------------------------------------------------- RMSNorm

RMS_MAX_K = 4096


def _rows(t: Tensor, K: int) -> Tensor:
    """``t [..., K]`` as an ``[M, K]`` row view (copied only if its layout does not fit the
    kernels: unit inner stride, 16-byte aligned base, row stride a multiple of 8)."""
    t2 = t.reshape(-1, K)
    ok = t2.stride(-1) == 1 and t2.data_ptr() % 16 == 0 and (t2.size(0) <= 1 or t2.stride(0) % 8 == 0)
    return t2 if ok else t2.contiguous()


def _rms_check(op: str, x: Tensor, weight: Tensor) -> int:
    _require_gpu(op, x, weight)
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"{op}: x must be bfloat16 or float32, got {x.dtype}")
    K = x.size(-1)
    if weight.shape != (K,):
        raise ValueError(f"{op}: weight must be [{K}], got {tuple(weight.shape)}")
    if K % 8 or K > RMS_MAX_K or K == 0:
        raise ValueError(f"{op}: last dim {K} must be a positive multiple of 8 and at most {RMS_MAX_K}")
    return K


def _dt_code(t: Tensor) -> int:
    return _lib.MLA_DTYPE_F32 if t.dtype == torch.float32 else _lib.MLA_DTYPE_BF16


@_op("rmsnorm", mutates_args=())
def rmsnorm(x: Tensor, weight: Tensor, eps: float, out_fp32: bool = False) -> Tuple[Tensor, Tensor]:
    """RMSNorm over the last dim (RMSNorm.forward, transformer.py:26-27):
    ``y = (x * r) * weight`` with ``r = 1 / sqrt(mean(x^2) + eps)`` in fp32.

    Returns ``y`` (x's shape; bf16, or fp32 when ``out_fp32``) and ``r`` (fp32, x's shape
    without the last dim).  The bf16 rounding is the one autocast applies where the
    down-projection GEMMs read the norm's output (transformer.py:338 -> :208-213); an fp32
    module outside autocast keeps the fp32 result."""
    op = "mla_mi355x::rmsnorm"
    K = _rms_check(op, x, weight)
    xr = _rows(x, K)
    M = xr.size(0)
    w = weight.detach().to(torch.float32).contiguous()
    y = torch.empty(M, K, dtype=torch.float32 if out_fp32 else torch.bfloat16, device=x.device)
    inv = torch.empty(M, dtype=torch.float32, device=x.device)
    if M:
        args = _lib.RmsNormArgs(
            x=xr.data_ptr(), w=w.data_ptr(), y=y.data_ptr(), inv_rms=inv.data_ptr(), M=M, K=K,
            x_stride=xr.stride(0) if M > 1 else K, y_stride=K, eps=float(eps), x_dtype=_dt_code(x),
            y_dtype=_dt_code(y))
        _lib.check(_lib.entry("mla_rmsnorm")(ctypes.byref(args), _stream(y)), op)
    return y.view(x.shape), inv.view(x.shape[:-1])


@rmsnorm.register_fake
def _(x, weight, eps, out_fp32=False):
    return (x.new_empty(x.shape, dtype=torch.float32 if out_fp32 else torch.bfloat16),
            x.new_empty(x.shape[:-1], dtype=torch.float32))


NORM_LINEAR_MAX_K = 4096


@_op("norm_linear", mutates_args=())
def norm_linear(x: Tensor, weight: Tensor, w_norm: Tensor, eps: float) -> Tuple[Tensor, Tensor]:
    """RMSNorm fused into a linear layer (the block's norm1 feeding the down-projections,
    transformer.py:26-27 and :338 -> :208-213): ``y = bf16(bf16((x * r) * w_norm) @ weight^T)`` with
    ``r = 1 / sqrt(mean(x^2) + eps)`` in fp32, for bf16 ``x [..., K]``, bf16 ``weight [N, K]``
    (nn.Linear layout) and ``w_norm [K]``; the normalised rows are never stored.  Returns ``y``
    (``x``'s leading dims, N) and ``r`` (fp32, ``x``'s leading dims).  K a multiple of 32 up to
    4096, N a multiple of 4."""
    op = "mla_mi355x::norm_linear"
    _require_gpu(op, x, weight, w_norm)
    _bf16(op, x=x, weight=weight)
    K = x.size(-1)
    if weight.dim() != 2 or weight.size(1) != K or w_norm.shape != (K,):
        raise ValueError(f"{op}: expected x [..., K], weight [N, K], w_norm [K]; got {tuple(x.shape)}, "
                         f"{tuple(weight.shape)}, {tuple(w_norm.shape)}")
    N = weight.size(0)
    if K % 32 or K > NORM_LINEAR_MAX_K or K == 0 or N % 4:
        raise ValueError(f"{op}: K = {K} must be a positive multiple of 32 up to {NORM_LINEAR_MAX_K} and "
                         f"N = {N} a multiple of 4")
    xr = _rows(x, K)
    M = xr.size(0)
    w = weight if (weight.stride(1) == 1 and weight.stride(0) % 8 == 0 and weight.data_ptr() % 16 == 0) \
        else weight.contiguous()
    wn = w_norm.detach().to(torch.float32).contiguous()
    y = torch.empty(M, N, dtype=torch.bfloat16, device=x.device)
    inv = torch.empty(M, dtype=torch.float32, device=x.device)
    if M and N:
        args = _lib.NormLinearArgs(
            x=xr.data_ptr(), w=w.data_ptr(), w_norm=wn.data_ptr(), y=y.data_ptr(), inv_rms=inv.data_ptr(), M=M, N=N,
            K=K, x_stride=xr.stride(0) if M > 1 else K, w_stride=w.stride(0) if N > 1 else K, y_stride=N,
            eps=float(eps))
        _lib.check(_lib.entry("mla_norm_linear")(ctypes.byref(args), _stream(y)), op)
    return y.view(*x.shape[:-1], N), inv.view(x.shape[:-1])


@norm_linear.register_fake
def _(x, weight, w_norm, eps):
    return x.new_empty(*x.shape[:-1], weight.size(0)), x.new_empty(x.shape[:-1], dtype=torch.float32)


@_op("rmsnorm_bwd", mutates_args=())
def rmsnorm_bwd(dy: Tensor, x: Tensor, weight: Tensor, inv_rms: Tensor) -> Tuple[Tensor, Tensor]:
    """Gradients ``(dx, dw)`` of :func:`rmsnorm` (the autograd of transformer.py:26-27):
    ``dx = r g - x r^3 / K sum(g x)`` with ``g = weight dy``, and ``dw = sum_rows dy x r``
    (fp32, summed in a fixed order).  ``dx`` has x's dtype; ``dy`` is read as bf16 or fp32."""
    op = "mla_mi355x::rmsnorm_bwd"
    K = _rms_check(op, x, weight)
    _require_gpu(op, dy, inv_rms)
    if dy.shape != x.shape or inv_rms.shape != x.shape[:-1] or inv_rms.dtype != torch.float32:
        raise ValueError(f"{op}: dy must match x {tuple(x.shape)} and inv_rms be fp32 {tuple(x.shape[:-1])}")
    xr = _rows(x, K)
    dyr = _rows(dy if dy.dtype in (torch.bfloat16, torch.float32) else dy.float(), K)
    inv = inv_rms.reshape(-1).contiguous()
    M = xr.size(0)
    w = weight.detach().to(torch.float32).contiguous()
    dx = torch.empty(M, K, dtype=x.dtype, device=x.device)
    dw = torch.empty(K, dtype=torch.float32, device=x.device)
    args = _lib.RmsNormBwdArgs(
        dy=dyr.data_ptr(), x=xr.data_ptr(), w=w.data_ptr(), inv_rms=inv.data_ptr(), dx=dx.data_ptr(),
        dw=dw.data_ptr(), workspace=None, workspace_bytes=0, M=M, K=K,
        dy_stride=dyr.stride(0) if M > 1 else K, x_stride=xr.stride(0) if M > 1 else K, dx_stride=K,
        x_dtype=_dt_code(x), dy_dtype=_dt_code(dyr))
    nbytes = int(_lib.entry("mla_rmsnorm_bwd_workspace_bytes")(ctypes.byref(args)))
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=x.device)
    args.workspace = ws.data_ptr()
    args.workspace_bytes = nbytes
    _lib.check(_lib.entry("mla_rmsnorm_bwd")(ctypes.byref(args), _stream(dx)), op)
    return dx.view(x.shape), dw


@rmsnorm_bwd.register_fake
def _(dy, x, weight, inv_rms):
    return torch.empty_like(x, memory_format=torch.contiguous_format), x.new_empty(x.size(-1), dtype=torch.float32)


def _rms_setup(ctx, inputs, output):
    x, weight, eps, out_fp32 = inputs
    ctx.save_for_backward(x, weight, output[1])
    ctx.mark_non_differentiable(output[1])


def _rms_backward(ctx, dy, dinv):
    x, weight, inv = ctx.saved_tensors
    dx, dw = torch.ops.mla_mi355x.rmsnorm_bwd(dy, x, weight, inv)
    return dx, dw.to(weight.dtype), None, None


rmsnorm.register_autograd(_rms_backward, setup_context=_rms_setup)


# ----------------------------------------------------------------- chunked linear cross-entropy

def _ce_check(op: str, logits: Tensor, targets: Tensor, lse: Tensor) -> Tuple[int, int]:
    _require_gpu(op, logits, targets, lse)
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"{op}: logits must be bfloat16 or float32, got {logits.dtype}")
    if logits.dim() != 2 or logits.stride(-1) != 1 or logits.data_ptr() % 16 or logits.size(1) % 8 \
            or (logits.size(0) > 1 and logits.stride(0) % 8):
        raise ValueError(f"{op}: logits must be [N, Vc] with Vc a multiple of 8, unit inner stride, 16-byte aligned "
                         "rows (row stride a multiple of 8)")
    N, Vc = logits.shape
    if targets.dtype != torch.int64 or tuple(targets.shape) != (N,) or not targets.is_contiguous():
        raise ValueError(f"{op}: targets must be a contiguous int64 [N]")
    if lse.dtype != torch.float32 or tuple(lse.shape) != (N,) or not lse.is_contiguous():
        raise ValueError(f"{op}: lse must be a contiguous fp32 [N]")
    return N, Vc


@_op("ce_chunk_fwd", mutates_args=("lse", "tlogit"))
def ce_chunk_fwd(logits: Tensor, targets: Tensor, lse: Tensor, tlogit: Tensor, v0: int) -> None:
    """One vocabulary chunk of chunked_linear_cross_entropy (transformer.py:91-108): folds the
    chunk's fp32 log-sum-exp into ``lse`` and gathers the target logit into ``tlogit`` for the
    rows whose target lies in ``[v0, v0 + Vc)``."""
    op = "mla_mi355x::ce_chunk_fwd"
    N, Vc = _ce_check(op, logits, targets, lse)
    if tlogit.dtype != torch.float32 or tuple(tlogit.shape) != (N,) or not tlogit.is_contiguous():
        raise ValueError(f"{op}: tlogit must be a contiguous fp32 [N]")
    args = _lib.CeChunkArgs(logits=logits.data_ptr(), dlogits=None, targets=targets.data_ptr(), lse=lse.data_ptr(),
                            tlogit=tlogit.data_ptr(), g_vec=None, g_scale=1.0, backward=0, N=N, Vc=Vc, v0=int(v0),
                            ld=logits.stride(0) if N > 1 else Vc, ld_out=0, dtype=_dt_code(logits))
    _lib.check(_lib.entry("mla_ce_chunk")(ctypes.byref(args), _stream(lse)), op)


@ce_chunk_fwd.register_fake
def _(logits, targets, lse, tlogit, v0):
    return None


@_op("ce_chunk_bwd_", mutates_args=("logits",))
def ce_chunk_bwd_(logits: Tensor, targets: Tensor, lse: Tensor, g_vec: Optional[Tensor], g_scale: float,
                  v0: int) -> None:
    """In place: ``logits <- g (softmax(logits) - onehot(target - v0))`` over one vocabulary
    chunk, with the final ``lse`` and ``g = g_scale * g_vec`` (or ``g_scale``) per row (the
    gradient of the loss with respect to the chunk's logits)."""
    op = "mla_mi355x::ce_chunk_bwd_"
    N, Vc = _ce_check(op, logits, targets, lse)
    if g_vec is not None and (g_vec.dtype != torch.float32 or tuple(g_vec.shape) != (N,) or not g_vec.is_contiguous()):
        raise ValueError(f"{op}: g_vec must be a contiguous fp32 [N]")
    ld = logits.stride(0) if N > 1 else Vc
    args = _lib.CeChunkArgs(logits=logits.data_ptr(), dlogits=logits.data_ptr(), targets=targets.data_ptr(),
                            lse=lse.data_ptr(), tlogit=None, g_vec=_ptr(g_vec), g_scale=float(g_scale), backward=1,
                            N=N, Vc=Vc, v0=int(v0), ld=ld, ld_out=ld, dtype=_dt_code(logits))
    _lib.check(_lib.entry("mla_ce_chunk")(ctypes.byref(args), _stream(lse)), op)


@ce_chunk_bwd_.register_fake
def _(logits, targets, lse, g_vec, g_scale, v0):
    return None


# ----------------------------------------------------------------- eager calls

def dispatcher_needed(args) -> bool:
    """Whether a call with ``args`` must go through the registered operator: under tracing
    (torch.compile), a dispatch mode (fake tensors, functionalization), a functorch transform,
    tensor subclasses, tensors off the GPU (meta tensors take the fake kernels), or an input
    that needs a gradient while grad mode is on (the autograd formulas live on the
    operators).  Otherwise the operator adds only dispatch time (about 15 us of Python per
    call) around the same body."""
    if torch.compiler.is_compiling() or torch._C._len_torch_dispatch_stack() > 0 \
            or torch._C._functorch.peek_interpreter_stack() is not None:
        return True
    grad = torch.is_grad_enabled()
    for a in args:
        if isinstance(a, Tensor):
            if (type(a) is not Tensor and type(a) is not torch.nn.Parameter) or not a.is_cuda:
                return True
            if grad and a.requires_grad:
                return True
    return False


def _eager_call(name: str):
    body = _BODIES[name]
    op = getattr(torch.ops.mla_mi355x, name)

    def call(*args, **kwargs):
        if dispatcher_needed(args) or (kwargs and dispatcher_needed(kwargs.values())):
            return op(*args, **kwargs)
        return body(*args, **kwargs)

    call.__name__ = name
    call.__doc__ = body.__doc__
    return call


class _EagerOps:
    """``torch.ops.mla_mi355x`` for eager callers: each attribute runs the operator's own body
    directly when ``dispatcher_needed`` is false, else the registered operator."""

    def __init__(self):
        for name in _BODIES:
            setattr(self, name, _eager_call(name))


eager = _EagerOps()
