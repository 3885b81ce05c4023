"""ctypes binding of the C ABI in ``include/mla_mi355x.h`` (libmla_mi355x.so).

The structs below mirror the header field for field; ``check_abi()`` compares
their sizes with the library's own ``mla_args_size``.  Loading fails loudly if
the library has not been built: there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import os
import threading
from ctypes import c_float, c_int, c_int32, c_int64, c_size_t, c_void_p, POINTER

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmla_mi355x.so")

MLA_OK = 0
MLA_ERR_INVALID_ARG = -1
MLA_ERR_UNSUPPORTED = -2
MLA_ERR_WORKSPACE = -3
MLA_ERR_LAUNCH = -4
MLA_DTYPE_BF16 = 0
MLA_DTYPE_F32 = 1
MLA_DECODE_STATIC_SCRATCH_BYTES = 12 << 20
ABI_VERSION = 3


class Strides(ctypes.Structure):
    _fields_ = [("b", c_int64), ("t", c_int64), ("h", c_int64)]


class RopeArgs(ctypes.Structure):
    _fields_ = [
        ("x", c_void_p), ("y", c_void_p), ("cos", c_void_p), ("sin", c_void_p),
        ("B", c_int64), ("T", c_int64), ("n_heads", c_int64), ("table_rows", c_int64), ("pos_offset", c_int64),
        ("x_stride", Strides), ("y_stride", Strides),
        ("dtype", c_int32), ("inverse", c_int32),
    ]


class RopeAppendArgs(ctypes.Structure):
    _fields_ = [
        ("qk", c_void_p), ("q_out", c_void_p), ("c_new", c_void_p), ("latent", c_void_p), ("k_cache", c_void_p),
        ("cos", c_void_p), ("sin", c_void_p), ("pos_dev", c_void_p), ("seq_lens", c_void_p), ("pos_next", c_void_p),
        ("B", c_int64), ("T", c_int64), ("H", c_int64), ("Hr", c_int64), ("d_latent", c_int64),
        ("capacity", c_int64), ("table_rows", c_int64), ("pos_offset", c_int64),
        ("qk_stride", Strides), ("q_stride", Strides),
        ("c_new_sb", c_int64), ("c_new_st", c_int64), ("latent_sb", c_int64), ("latent_st", c_int64),
        ("k_cache_sb", c_int64), ("k_cache_sh", c_int64), ("k_cache_st", c_int64),
    ]


class PrefillFwdArgs(ctypes.Structure):
    _fields_ = [
        ("q_nope", c_void_p), ("q_rope", c_void_p), ("k_nope", c_void_p), ("k_rope", c_void_p), ("v", c_void_p),
        ("o", c_void_p), ("lse", c_void_p),
        ("B", c_int64), ("H", c_int64), ("Tq", c_int64), ("Tk", c_int64),
        ("d_nope", c_int64), ("d_rope", c_int64), ("d_v", c_int64),
        ("q_nope_stride", Strides), ("q_rope_stride", Strides), ("k_nope_stride", Strides),
        ("k_rope_stride", Strides), ("v_stride", Strides), ("o_stride", Strides),
        ("scale", c_float), ("causal", c_int32), ("q_offset", c_int64),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
        ("rope_cos", c_void_p), ("rope_sin", c_void_p), ("rope_rows", c_int64), ("q_pos_offset", c_int64),
        ("q_rope_out", c_void_p), ("q_rope_out_stride", Strides),
    ]


class PrefillBwdArgs(ctypes.Structure):
    _fields_ = [
        ("dout", c_void_p), ("q_nope", c_void_p), ("q_rope", c_void_p), ("k_nope", c_void_p), ("k_rope", c_void_p),
        ("v", c_void_p), ("o", c_void_p), ("lse", c_void_p),
        ("dq_nope", c_void_p), ("dq_rope", c_void_p), ("dk_nope", c_void_p), ("dk_rope", c_void_p), ("dv", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
        ("B", c_int64), ("H", c_int64), ("Tq", c_int64), ("Tk", c_int64),
        ("d_nope", c_int64), ("d_rope", c_int64), ("d_v", c_int64),
        ("dout_stride", Strides), ("q_nope_stride", Strides), ("q_rope_stride", Strides), ("k_nope_stride", Strides),
        ("k_rope_stride", Strides), ("v_stride", Strides), ("o_stride", Strides),
        ("dq_nope_stride", Strides), ("dq_rope_stride", Strides), ("dk_nope_stride", Strides),
        ("dk_rope_stride", Strides), ("dv_stride", Strides),
        ("scale", c_float), ("causal", c_int32), ("q_offset", c_int64),
        ("rope_cos", c_void_p), ("rope_sin", c_void_p), ("rope_rows", c_int64), ("q_pos_offset", c_int64),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("q_lat", c_void_p), ("q_rope", c_void_p), ("c_kv", c_void_p), ("k_rope", c_void_p),
        ("seq_lens", c_void_p), ("ctx", c_void_p), ("lse", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t),
        ("B", c_int64), ("H", c_int64), ("L", c_int64), ("d_latent", c_int64), ("d_rope", c_int64),
        ("n_k_rope_heads", c_int64),
        ("q_lat_sb", c_int64), ("q_lat_sh", c_int64), ("q_rope_sb", c_int64), ("q_rope_sh", c_int64),
        ("c_kv_sb", c_int64), ("c_kv_st", c_int64),
        ("k_rope_sb", c_int64), ("k_rope_sh", c_int64), ("k_rope_st", c_int64),
        ("ctx_sb", c_int64), ("ctx_sh", c_int64),
        ("scale", c_float), ("num_splits", c_int32),
    ]


class DecodeOutArgs(ctypes.Structure):
    _fields_ = [
        ("dec", DecodeArgs), ("w_uv", c_void_p), ("out", c_void_p),
        ("w_uv_sh", c_int64), ("w_uv_sd", c_int64), ("out_sb", c_int64), ("out_sh", c_int64), ("d_v", c_int64),
    ]


class NormLinearArgs(ctypes.Structure):
    _fields_ = [
        ("x", c_void_p), ("w", c_void_p), ("w_norm", c_void_p), ("y", c_void_p), ("inv_rms", c_void_p),
        ("M", c_int64), ("N", c_int64), ("K", c_int64), ("x_stride", c_int64), ("w_stride", c_int64),
        ("y_stride", c_int64), ("eps", c_float),
    ]


class PrefillCachedArgs(ctypes.Structure):
    _fields_ = [
        ("q_lat", c_void_p), ("q_rope", c_void_p), ("c_kv", c_void_p), ("k_rope", c_void_p),
        ("ctx", c_void_p), ("lse", c_void_p), ("workspace", c_void_p), ("workspace_bytes", c_size_t),
        ("B", c_int64), ("T", c_int64), ("H", c_int64), ("L", c_int64), ("L0", c_int64),
        ("d_latent", c_int64), ("d_rope", c_int64),
        ("q_lat_stride", Strides), ("q_rope_stride", Strides), ("ctx_stride", Strides),
        ("c_kv_sb", c_int64), ("c_kv_st", c_int64), ("k_rope_sb", c_int64), ("k_rope_st", c_int64),
        ("scale", c_float), ("num_splits", c_int32),
    ]


class AbsorbQArgs(ctypes.Structure):
    _fields_ = [
        ("q_nope", c_void_p), ("w_uk", c_void_p), ("q_lat", c_void_p),
        ("B", c_int64), ("H", c_int64), ("d_nope", c_int64), ("d_latent", c_int64),
        ("q_sb", c_int64), ("q_sh", c_int64), ("w_uk_sh", c_int64), ("w_uk_sd", c_int64),
        ("out_sb", c_int64), ("out_sh", c_int64),
    ]


class CeChunkArgs(ctypes.Structure):
    _fields_ = [
        ("logits", c_void_p), ("dlogits", c_void_p), ("targets", c_void_p), ("lse", c_void_p), ("tlogit", c_void_p),
        ("g_vec", c_void_p), ("g_scale", c_float), ("backward", c_int32),
        ("N", c_int64), ("Vc", c_int64), ("v0", c_int64), ("ld", c_int64), ("ld_out", c_int64),
        ("dtype", c_int32),
    ]


class LinearRowsArgs(ctypes.Structure):
    _fields_ = [
        ("x", c_void_p), ("w", c_void_p), ("y", c_void_p),
        ("M", c_int64), ("N", c_int64), ("K", c_int64), ("G", c_int64),
        ("x_sm", c_int64), ("x_sg", c_int64), ("w_sn", c_int64), ("w_sg", c_int64), ("y_sm", c_int64), ("y_sg", c_int64),
    ]


class RmsNormArgs(ctypes.Structure):
    _fields_ = [
        ("x", c_void_p), ("w", c_void_p), ("y", c_void_p), ("inv_rms", c_void_p),
        ("M", c_int64), ("K", c_int64), ("x_stride", c_int64), ("y_stride", c_int64),
        ("eps", c_float), ("x_dtype", c_int32), ("y_dtype", c_int32),
    ]


class RmsNormBwdArgs(ctypes.Structure):
    _fields_ = [
        ("dy", c_void_p), ("x", c_void_p), ("w", c_void_p), ("inv_rms", c_void_p),
        ("dx", c_void_p), ("dw", c_void_p), ("workspace", c_void_p), ("workspace_bytes", c_size_t),
        ("M", c_int64), ("K", c_int64), ("dy_stride", c_int64), ("x_stride", c_int64), ("dx_stride", c_int64),
        ("x_dtype", c_int32), ("dy_dtype", c_int32),
    ]


ARGS_STRUCTS = {0: RopeArgs, 1: PrefillFwdArgs, 2: PrefillBwdArgs, 3: DecodeArgs, 4: RmsNormArgs,
                5: RmsNormBwdArgs, 6: DecodeOutArgs, 7: RopeAppendArgs, 8: AbsorbQArgs, 9: CeChunkArgs,
                10: LinearRowsArgs, 11: PrefillCachedArgs, 12: NormLinearArgs}

# exported symbol -> (restype, argtypes)
SIGNATURES = {
    "mla_rope": (c_int, [POINTER(RopeArgs), c_void_p]),
    "mla_rope_append": (c_int, [POINTER(RopeAppendArgs), c_void_p]),
    "mla_prefill_fwd_workspace_bytes": (c_size_t, [POINTER(PrefillFwdArgs)]),
    "mla_prefill_fwd": (c_int, [POINTER(PrefillFwdArgs), c_void_p]),
    "mla_prefill_bwd_workspace_bytes": (c_size_t, [POINTER(PrefillBwdArgs)]),
    "mla_prefill_bwd_workspace_min_bytes": (c_size_t, [POINTER(PrefillBwdArgs)]),
    "mla_prefill_bwd": (c_int, [POINTER(PrefillBwdArgs), c_void_p]),
    "mla_decode_workspace_bytes": (c_size_t, [POINTER(DecodeArgs)]),
    "mla_decode": (c_int, [POINTER(DecodeArgs), c_void_p]),
    "mla_decode_static": (c_int, [POINTER(DecodeArgs), c_void_p]),
    "mla_absorb_q": (c_int, [POINTER(AbsorbQArgs), c_void_p]),
    "mla_norm_linear": (c_int, [POINTER(NormLinearArgs), c_void_p]),
    "mla_prefill_cached_workspace_bytes": (c_size_t, [POINTER(PrefillCachedArgs)]),
    "mla_prefill_cached": (c_int, [POINTER(PrefillCachedArgs), c_void_p]),
    "mla_decode_out_workspace_bytes": (c_size_t, [POINTER(DecodeOutArgs)]),
    "mla_decode_out": (c_int, [POINTER(DecodeOutArgs), c_void_p]),
    "mla_ce_chunk": (c_int, [POINTER(CeChunkArgs), c_void_p]),
    "mla_linear_rows": (c_int, [POINTER(LinearRowsArgs), c_void_p]),
    "mla_linear_rows_rope_append": (c_int, [POINTER(LinearRowsArgs), POINTER(RopeAppendArgs), c_void_p]),
    "mla_rmsnorm": (c_int, [POINTER(RmsNormArgs), c_void_p]),
    "mla_rmsnorm_bwd_workspace_bytes": (c_size_t, [POINTER(RmsNormBwdArgs)]),
    "mla_rmsnorm_bwd": (c_int, [POINTER(RmsNormBwdArgs), c_void_p]),
    "mla_last_error": (ctypes.c_char_p, []),
    "mla_abi_version": (c_int, []),
    "mla_args_size": (c_size_t, [c_int]),
}

_lib = None
_lock = threading.Lock()


class MLAKernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(path):
                raise RuntimeError(
                    f"transformer_amd: HIP library {path} is not built; run "
                    "`python -m transformer_amd.build` (or __graft_entry__.build()). "
                    "There is no fallback implementation.")
            lib = ctypes.CDLL(path)
            missing = []
            for name, (res, args) in SIGNATURES.items():
                try:
                    fn = getattr(lib, name)
                except AttributeError:
                    missing.append(name)
                    continue
                fn.restype = res
                fn.argtypes = args
            lib.missing_symbols = missing
            _lib = lib
            check_abi()
    return _lib


def check_abi() -> None:
    lib = _lib
    if lib.mla_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libmla_mi355x ABI {lib.mla_abi_version()} != binding ABI {ABI_VERSION}")
    for which, st in ARGS_STRUCTS.items():
        n = lib.mla_args_size(which)
        if n != ctypes.sizeof(st):
            raise RuntimeError(f"ABI mismatch for {st.__name__}: library {n} bytes, binding {ctypes.sizeof(st)}")


def entry(name: str):
    """Return the bound C entry point ``name``; raises if the library lacks it."""
    lib = load()
    if name in lib.missing_symbols:
        raise RuntimeError(f"libmla_mi355x.so does not export {name}; rebuild the library")
    return getattr(lib, name)


def check(rc: int, op: str) -> None:
    if rc != MLA_OK:
        msg = _lib.mla_last_error().decode(errors="replace")
        raise MLAKernelError(f"{op} failed ({rc}): {msg}")
