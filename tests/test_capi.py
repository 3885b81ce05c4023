"""CPU-side checks of the C-ABI boundary: the built library loads, exports every
symbol declared in include/*.h, and its argument-struct sizes match the ctypes
binding.  No kernel is launched (there is no GPU here)."""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(mla_[a-z0-9_]+)\s*\(", text, re.M):
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def lib():
    from transformer_amd import _lib
    return _lib.load()


def test_header_declares_the_entry_points():
    names = declared_symbols()
    for n in ("mla_rope", "mla_prefill_fwd", "mla_prefill_bwd", "mla_prefill_bwd_workspace_bytes", "mla_decode",
              "mla_decode_workspace_bytes", "mla_last_error", "mla_abi_version", "mla_args_size"):
        assert n in names, n


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing
    assert not lib.missing_symbols


def test_binding_covers_every_declared_symbol():
    from transformer_amd import _lib
    assert declared_symbols() <= set(_lib.SIGNATURES)


def test_struct_sizes_match(lib):
    from transformer_amd import _lib
    for which, st in _lib.ARGS_STRUCTS.items():
        assert lib.mla_args_size(which) == ctypes.sizeof(st), st.__name__
    assert lib.mla_abi_version() == _lib.ABI_VERSION


def test_invalid_arguments_are_rejected_without_a_gpu(lib):
    # argument validation runs on the host before any launch
    from transformer_amd import _lib
    a = _lib.PrefillFwdArgs()
    a.d_nope, a.d_rope, a.d_v, a.scale = 96, 64, 128, 0.125
    rc = lib.mla_prefill_fwd(ctypes.byref(a), None)
    assert rc == _lib.MLA_ERR_UNSUPPORTED
    assert b"not built" in lib.mla_last_error()
    r = _lib.RopeArgs()
    r.x = r.y = r.cos = r.sin = 16
    r.B, r.T, r.n_heads, r.table_rows, r.pos_offset = 1, 8, 1, 4, 0
    assert lib.mla_rope(ctypes.byref(r), None) == _lib.MLA_ERR_INVALID_ARG
    assert b"exceed" in lib.mla_last_error()
    # the kernel's index arithmetic is 32-bit: 2^31 or more head vectors are refused
    r.B, r.T, r.n_heads, r.table_rows = 1 << 20, 1 << 10, 2, 1 << 20
    assert lib.mla_rope(ctypes.byref(r), None) == _lib.MLA_ERR_INVALID_ARG
    assert b"too many vectors" in lib.mla_last_error()
    r.B, r.T, r.n_heads = 1 << 40, 1 << 10, 1 << 20
    assert lib.mla_rope(ctypes.byref(r), None) == _lib.MLA_ERR_INVALID_ARG
    assert b"overflows" in lib.mla_last_error()
    d = _lib.DecodeArgs()
    d.B, d.H, d.L, d.d_latent, d.d_rope, d.n_k_rope_heads, d.scale = 1, 16, 0, 512, 64, 1, 0.125
    assert lib.mla_decode(ctypes.byref(d), None) == _lib.MLA_ERR_INVALID_ARG
    assert b"L = 0" in lib.mla_last_error()
    assert lib.mla_decode_workspace_bytes(ctypes.byref(d)) == 0


def test_decode_workspace_query(lib):
    from transformer_amd import _lib
    d = _lib.DecodeArgs()
    d.B, d.H, d.L, d.d_latent, d.d_rope, d.n_k_rope_heads, d.num_splits = 32, 16, 4096, 512, 64, 1, 16
    # 16 splits: partial outputs [32][16][16][512] bf16 + LSEs [32][16][16] fp32
    assert lib.mla_decode_workspace_bytes(ctypes.byref(d)) >= 32 * 16 * 16 * 512 * 2 + 32 * 16 * 16 * 4
    d.num_splits = 1
    assert lib.mla_decode_workspace_bytes(ctypes.byref(d)) == 0


def test_cpu_tensors_fail_loudly():
    import torch
    import transformer_amd  # noqa: F401
    x = torch.zeros(1, 4, 1, 64, dtype=torch.bfloat16)
    c = torch.zeros(8, 32, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        torch.ops.mla_mi355x.rope(x, c, c, 0, False)


def test_new_entry_points_reject_invalid_arguments_without_a_gpu(lib):
    # every check below runs on the host before any launch
    from transformer_amd import _lib
    r = _lib.RmsNormArgs()
    r.M, r.K, r.x_dtype = 4, 12, _lib.MLA_DTYPE_BF16  # K not a multiple of 8
    assert lib.mla_rmsnorm(ctypes.byref(r), None) == _lib.MLA_ERR_UNSUPPORTED
    r.K = 8192  # above the 4096 the kernels keep in registers
    assert lib.mla_rmsnorm(ctypes.byref(r), None) == _lib.MLA_ERR_UNSUPPORTED
    rb = _lib.RmsNormBwdArgs()
    rb.M, rb.K, rb.x_dtype, rb.w, rb.dw = 4, 64, _lib.MLA_DTYPE_BF16, 16, 16
    rb.dy = rb.x = rb.dx = 16
    rb.dy_stride = rb.x_stride = rb.dx_stride = 64
    rb.inv_rms = 16
    assert lib.mla_rmsnorm_bwd_workspace_bytes(ctypes.byref(rb)) == 1 * 64 * 4  # one workgroup's dw row
    assert lib.mla_rmsnorm_bwd(ctypes.byref(rb), None) == _lib.MLA_ERR_WORKSPACE  # none given
    o = _lib.DecodeOutArgs()
    d = o.dec
    d.B, d.H, d.L, d.d_latent, d.d_rope, d.n_k_rope_heads, d.scale = 2, 4, 64, 512, 64, 1, 0.125
    d.q_lat = d.q_rope = d.c_kv = d.k_rope = d.lse = 256
    o.w_uv = o.out = 256
    o.w_uv_sh, o.w_uv_sd, o.d_v = 96 * 512, 512, 96
    assert lib.mla_decode_out(ctypes.byref(o), None) == _lib.MLA_ERR_UNSUPPORTED  # d_v 96 not built
    ra = _lib.RopeAppendArgs()
    ra.qk = ra.q_out = ra.c_new = ra.latent = ra.k_cache = ra.cos = ra.sin = 256
    ra.B, ra.T, ra.H, ra.Hr, ra.d_latent, ra.capacity, ra.table_rows, ra.pos_offset = 1, 4, 2, 1, 64, 16, 64, 14
    assert lib.mla_rope_append(ctypes.byref(ra), None) == _lib.MLA_ERR_INVALID_ARG  # rows 14..17 past capacity 16
    assert b"exceed" in lib.mla_last_error()
    # the combined q_up + append launch runs both parts' checks before launching anything
    lr = _lib.LinearRowsArgs()
    lr.x = lr.w = lr.y = 256
    lr.M, lr.N, lr.K, lr.G, lr.x_sm, lr.w_sn, lr.y_sm = 32, 2048, 1000, 1, 1000, 1000, 2048  # K not a multiple of 128
    assert lib.mla_linear_rows_rope_append(ctypes.byref(lr), ctypes.byref(ra), None) == _lib.MLA_ERR_UNSUPPORTED
    assert b"mla_linear_rows_rope_append" in lib.mla_last_error()
    lr.K, lr.x_sm, lr.w_sn = 1024, 1024, 1024  # the product is fine; the append's positions are not
    assert lib.mla_linear_rows_rope_append(ctypes.byref(lr), ctypes.byref(ra), None) == _lib.MLA_ERR_INVALID_ARG
    assert b"exceed" in lib.mla_last_error()
    assert lib.mla_linear_rows_rope_append(None, ctypes.byref(ra), None) == _lib.MLA_ERR_INVALID_ARG
    aq = _lib.AbsorbQArgs()
    aq.B, aq.H, aq.d_nope, aq.d_latent = 2, 4, 96, 512
    assert lib.mla_absorb_q(ctypes.byref(aq), None) == _lib.MLA_ERR_UNSUPPORTED  # d_nope 96 not built
    ce = _lib.CeChunkArgs()
    ce.N, ce.Vc = 8, 100  # chunk width not a multiple of 8
    assert lib.mla_ce_chunk(ctypes.byref(ce), None) == _lib.MLA_ERR_INVALID_ARG
    ce.Vc, ce.dtype = 64, 7  # logits dtype outside bf16 / fp32
    assert lib.mla_ce_chunk(ctypes.byref(ce), None) == _lib.MLA_ERR_UNSUPPORTED
    r.K, r.y_dtype = 64, 5  # output dtype outside bf16 / fp32
    assert lib.mla_rmsnorm(ctypes.byref(r), None) == _lib.MLA_ERR_UNSUPPORTED


@pytest.mark.parametrize("scale", [0.0, -0.125, float("nan"), float("inf"), 3e38])
def test_bad_softmax_scales_are_rejected_without_a_gpu(lib, scale):
    # the kernels take a row's reference max before scaling, which is only right for a finite
    # positive scale: zero, negative, NaN, infinite and overflowing scales (scale * log2 e = inf)
    # are refused on the host, before any launch
    from transformer_amd import _lib
    a = _lib.PrefillFwdArgs()
    a.d_nope, a.d_rope, a.d_v, a.B, a.H, a.Tq, a.Tk, a.scale = 128, 64, 128, 1, 1, 8, 8, scale
    assert lib.mla_prefill_fwd(ctypes.byref(a), None) == _lib.MLA_ERR_INVALID_ARG
    assert b"scale" in lib.mla_last_error()
    b = _lib.PrefillBwdArgs()
    b.d_nope, b.d_rope, b.d_v, b.B, b.H, b.Tq, b.Tk, b.scale = 128, 64, 128, 1, 1, 8, 8, scale
    assert lib.mla_prefill_bwd(ctypes.byref(b), None) == _lib.MLA_ERR_INVALID_ARG
    assert b"scale" in lib.mla_last_error()
    d = _lib.DecodeArgs()
    d.B, d.H, d.L, d.d_latent, d.d_rope, d.n_k_rope_heads, d.scale = 1, 16, 64, 512, 64, 1, scale
    assert lib.mla_decode(ctypes.byref(d), None) == _lib.MLA_ERR_INVALID_ARG
    assert b"scale" in lib.mla_last_error()
    o = _lib.DecodeOutArgs()
    o.dec.B, o.dec.H, o.dec.L, o.dec.d_latent, o.dec.d_rope, o.dec.n_k_rope_heads = 1, 16, 64, 512, 64, 1
    o.dec.scale, o.d_v = scale, 128
    assert lib.mla_decode_out(ctypes.byref(o), None) == _lib.MLA_ERR_INVALID_ARG
    assert b"scale" in lib.mla_last_error()


def test_decode_static_rejects_a_split_count_beyond_its_scratch():
    # host-side check, before the static array is looked up: no GPU needed
    from transformer_amd import _lib
    d = _lib.DecodeArgs()
    d.B, d.H, d.L, d.d_latent, d.d_rope, d.n_k_rope_heads, d.scale, d.num_splits = 64, 16, 65536, 512, 64, 1, 0.1, 64
    d.q_lat = d.q_rope = d.c_kv = d.k_rope = d.ctx = d.lse = 256
    need = _lib.entry("mla_decode_workspace_bytes")(ctypes.byref(d))
    assert need > _lib.MLA_DECODE_STATIC_SCRATCH_BYTES
    assert _lib.entry("mla_decode_static")(ctypes.byref(d), None) == _lib.MLA_ERR_WORKSPACE
    assert b"static scratch" in _lib.load().mla_last_error()


def _fwd_args(B, H, Tq, Tk, causal=1, q_offset=0):
    from transformer_amd import _lib
    a = _lib.PrefillFwdArgs()
    a.B, a.H, a.Tq, a.Tk, a.d_nope, a.d_rope, a.d_v = B, H, Tq, Tk, 128, 64, 128
    a.scale, a.causal, a.q_offset = 0.07, causal, q_offset
    return a


def test_prefill_fwd_workspace_query_picks_the_key_split(lib):
    # host-side choice of mla_prefill_fwd: no split (0 bytes) when the mirrored q-tile pairs give more than 128
    # workgroups; else S segments per pair for ~256 workgroups (at most 8, at least 8 key tiles each), with
    # B H n_qt S 128 rows of fp32 partials (512 B) and log2 LSEs (4 B) in the workspace
    def ws(*a, **k):
        return lib.mla_prefill_fwd_workspace_bytes(ctypes.byref(_fwd_args(*a, **k)))
    rows = lambda B, H, n_qt, S: B * H * n_qt * S * 128
    assert ws(12, 16, 2048, 2048) == 0                       # config 1: 1536 workgroups
    assert ws(2, 16, 2048, 2048) == 0                        # 256 pairs
    assert ws(1, 16, 2048, 2048) == rows(1, 16, 16, 2) * 516  # the reference's prompt: 128 pairs, S = 2
    assert ws(1, 2, 1024, 1024) == rows(1, 2, 8, 4) * 516     # 8 pairs: S = min(32, 8, 36 tiles / 8) = 4
    assert ws(1, 4, 100, 3000, causal=0) == rows(1, 4, 1, 8) * 516  # one q-tile over 94 key tiles: S = 8
    assert ws(1, 16, 200, 200) == 0                          # 13 key tiles per pair: too few to split
    assert ws(0, 16, 2048, 2048) == 0 and ws(1, 16, 2048, 2048, q_offset=-1) == 0


def _segments(n_qt, BM, Tk, causal, q_offset, S):
    """The key split restated (prefill_fwd.hip fwd_split_of_pair / fwd_qtile_parts): per pair (qa, qb) of
    n_a + n_b = N key tiles, segment s covers [floor(s N / S), floor((s + 1) N / S))."""
    tiles = lambda qt: -(-(min(Tk, qt * BM + BM + q_offset) if causal else Tk) // 32)
    out = {}
    for r in range((n_qt + 1) // 2):
        qa, qb = n_qt - 1 - r, r
        n_a, n_b = tiles(qa), (0 if qa == qb else tiles(qb))
        N = n_a + n_b
        c = [s * N // S for s in range(S + 1)]
        for s in range(S):
            if c[s] < n_a:
                out.setdefault(qa, []).append((s, c[s], min(c[s + 1], n_a)))
            if n_b > 0 and c[s + 1] > n_a:
                out.setdefault(qb, []).append((s, max(c[s], n_a) - n_a, c[s + 1] - n_a))
        # the closed forms the kernels use for a q-tile's partial count and first slot
        parts_a = -(-(n_a * S) // N)
        parts_b = S + 1 - (-(-((n_a + 1) * S) // N))
        assert [x[0] for x in out[qa]] == list(range(parts_a))
        if n_b:
            assert [x[0] for x in out[qb]] == list(range(S - parts_b, S))
    return out, tiles


@pytest.mark.parametrize("n_qt,Tk,causal,q_offset,S", [
    (16, 2048, 1, 0, 2), (16, 2048, 1, 0, 4), (8, 1024, 1, 0, 4), (3, 1280, 1, 1000, 8), (3, 1333, 1, 1033, 8),
    (1, 3000, 0, 0, 8), (6, 700, 1, 0, 3), (5, 640, 1, 0, 3), (7, 900, 1, 17, 5)])
def test_key_split_segments_cover_every_key_tile_once(n_qt, Tk, causal, q_offset, S):
    # brute force over the segment formula: every q-tile's key tiles are covered exactly once, in key order,
    # by consecutive slots, and the closed-form partial counts and first slots match the enumeration
    out, tiles = _segments(n_qt, 128, Tk, causal, q_offset, S)
    for qt in range(n_qt):
        ranges = out[qt]
        assert ranges[0][1] == 0 and ranges[-1][2] == tiles(qt)
        for (s0, lo0, hi0), (s1, lo1, hi1) in zip(ranges, ranges[1:]):
            assert s1 == s0 + 1 and lo1 == hi0 and lo0 < hi0


def test_workspace_queries_answer_zero_for_sizes_the_entries_reject(lib):
    # the queries test the sizes before any arithmetic on them (a query over Tq, Tk near 2^30 once
    # overflowed the stored-dS prefix in 64-bit arithmetic)
    from transformer_amd import _lib
    b = _lib.PrefillBwdArgs()
    b.B, b.H, b.Tq, b.Tk, b.d_nope, b.d_rope, b.d_v, b.causal = 1, 1, (1 << 62), (1 << 62), 128, 64, 128, 0
    assert lib.mla_prefill_bwd_workspace_bytes(ctypes.byref(b)) == 0
    assert lib.mla_prefill_bwd_workspace_min_bytes(ctypes.byref(b)) == 0
    b.Tq, b.Tk, b.q_offset, b.causal = 4096, 4096, -5, 1  # causal with a negative offset
    assert lib.mla_prefill_bwd_workspace_bytes(ctypes.byref(b)) == 0
    b.q_offset = 0
    assert lib.mla_prefill_bwd_workspace_bytes(ctypes.byref(b)) > 0
    d = _lib.DecodeArgs()
    d.B, d.H, d.L, d.d_latent, d.d_rope, d.num_splits = 32, 16, 4096, 512, 64, 8
    assert lib.mla_decode_workspace_bytes(ctypes.byref(d)) > 0
    for field, value in (("L", 1 << 40), ("d_latent", 100), ("d_rope", 32), ("B", 1 << 20)):
        d2 = _lib.DecodeArgs.from_buffer_copy(d)
        setattr(d2, field, value)
        assert lib.mla_decode_workspace_bytes(ctypes.byref(d2)) == 0, field
    d.B, d.H, d.L, d.num_splits = 65535, 65535, (1 << 30) - 1, (1 << 30)  # a grid of 2^31 or more workgroups
    assert lib.mla_decode_workspace_bytes(ctypes.byref(d)) == 0
    r = _lib.RmsNormBwdArgs()
    r.M, r.K = 64, 2049  # K must be a multiple of 8
    assert lib.mla_rmsnorm_bwd_workspace_bytes(ctypes.byref(r)) == 0
    r.K = 2048
    assert lib.mla_rmsnorm_bwd_workspace_bytes(ctypes.byref(r)) > 0


def test_workspace_queries_on_random_sizes(lib):
    # pure host functions (nothing launches): random and extreme sizes, including every 64-bit
    # edge, give an answer without faulting, and no answer is a wrapped-around size (2^56 bytes or more)
    import random
    from transformer_amd import _lib
    edges = [0, 1, 31, 32, 33, 127, 128, 129, 512, 4096, (1 << 30) - 1, 1 << 30, (1 << 31) - 1, 1 << 31, 1 << 40,
             (1 << 62), -1, -(1 << 62)]
    rng = random.Random(11)
    queries = [(n, s, a) for n, (s, a) in _lib.SIGNATURES.items() if n.endswith("_bytes")]
    assert len(queries) >= 7

    def fill(obj):
        for name, ftype in obj._fields_:
            if ftype is ctypes.c_void_p:
                setattr(obj, name, rng.choice([None, 0x10000000]))
            elif ftype is ctypes.c_float:
                setattr(obj, name, 0.07)
            elif isinstance(ftype, type) and issubclass(ftype, ctypes.Structure):
                fill(getattr(obj, name))
            else:
                v = rng.choice(edges) if rng.random() < 0.7 else rng.randint(0, 5000)
                if ftype in (ctypes.c_int32, ctypes.c_int):
                    v = max(min(v, (1 << 31) - 1), -(1 << 31))
                setattr(obj, name, abs(v) if ftype is ctypes.c_size_t else v)

    for name, _, args in queries:
        f = getattr(lib, name)
        for _ in range(400):
            a = args[0]._type_()
            fill(a)
            assert f(ctypes.byref(a)) < (1 << 56), name
