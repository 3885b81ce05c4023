"""Pin the CPU oracle (oracle/mla_oracle.py) before trusting it as the checker.

Each test checks the oracle against something other than its own formula: the
reference's golden vectors (tests/golden/), a library routine (torch SDPA),
brute-force loops, closed forms or invariants chosen so that a dropped term,
wrong sign or transposed operand fails.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import mla_oracle as O
from tests.golden_io import bf16_from_bits


# ---------------------------------------------------------------- RoPE tables / rotation

def test_rope_tables_match_reference_golden(golden):
    cos, sin = O.rope_tables(64, 16384, 10000.0)
    rows = torch.from_numpy(golden.raw["rope.rows"])
    assert torch.equal(cos[rows].view(torch.int16), bf16_from_bits(golden.raw["rope.cos"]).view(torch.int16))
    assert torch.equal(sin[rows].view(torch.int16), bf16_from_bits(golden.raw["rope.sin"]).view(torch.int16))


def test_rope_tables_closed_form():
    cos, sin = O.rope_tables(64, 16384, 10000.0)
    p = np.arange(16384, dtype=np.float64)[:, None]
    i = np.arange(32, dtype=np.float64)[None, :]
    ang = p * 10000.0 ** (-2.0 * i / 64.0)
    for tab, ref in ((cos, np.cos(ang)), (sin, np.sin(ang))):
        got = tab.double().numpy()
        # bf16 has 8 significant bits: |err| <= 2^-8 |x| (+ fp32 angle error, which grows with p)
        err = np.abs(got - ref)
        tol = np.abs(ref) * 2.0 ** -8 + 2e-3 * (p / 16384.0) + 1e-6
        assert (err <= tol).all()
        # and equals the correctly rounded bf16 of the exact value almost everywhere
        rounded = torch.from_numpy(ref).to(torch.bfloat16).double().numpy()
        assert (got[:2048] == rounded[:2048]).mean() > 0.98


def test_apply_rope_matches_reference_golden(golden):
    x = golden.t("rope.x")
    cos, sin = O.rope_tables(64, 64, 10000.0)
    y = O.apply_rope(x, cos.float(), sin.float())
    torch.testing.assert_close(y, golden.t("rope.y"), rtol=0, atol=1e-6)


def test_apply_rope_is_complex_rotation():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, 40, 64, generator=g, dtype=torch.float64)
    p = torch.arange(40, dtype=torch.float64)[:, None]
    ang = p * 10000.0 ** (-torch.arange(32, dtype=torch.float64) * 2 / 64)
    y = O.apply_rope(x, ang.cos(), ang.sin())
    z = torch.complex(x[..., :32], x[..., 32:]) * torch.exp(1j * ang)
    torch.testing.assert_close(y, torch.cat([z.real, z.imag], -1), rtol=1e-12, atol=1e-12)


def test_apply_rope_inverse_and_norm():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(3, 30, 64, generator=g, dtype=torch.float64)
    cos, sin = O.rope_tables(64, 30, 10000.0)
    c, s = cos.double(), sin.double()
    y = O.apply_rope(x, c, s)
    # per-pair norm is preserved up to the bf16 rounding of (c, s): c^2 + s^2 = 1 + O(2^-8)
    n0 = x[..., :32] ** 2 + x[..., 32:] ** 2
    n1 = y[..., :32] ** 2 + y[..., 32:] ** 2
    torch.testing.assert_close(n1 / (c * c + s * s), n0, rtol=1e-10, atol=1e-10)
    back = O.apply_rope(y, c, -s) / (c * c + s * s).repeat(1, 2)
    torch.testing.assert_close(back, x, rtol=1e-10, atol=1e-10)


def test_rope_relative_position_invariance():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(64, generator=g, dtype=torch.float64)
    k = torch.randn(64, generator=g, dtype=torch.float64)
    inv = 10000.0 ** (-torch.arange(32, dtype=torch.float64) * 2 / 64)

    def rot(x, p):
        a = p * inv
        return O.apply_rope(x.view(1, 64), a.cos().view(1, 32), a.sin().view(1, 32)).view(64)

    for p, pp in ((0, 5), (7, 12), (100, 105), (3, 1000)):
        assert abs(rot(q, p) @ rot(k, pp) - q @ rot(k, pp - p)) < 1e-10


# ---------------------------------------------------------------- attention (prefill)

def _qkv(B=2, H=3, Tq=17, Tk=17, D=24, Dv=16, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, H, Tq, D, generator=g, dtype=dtype),
            torch.randn(B, H, Tk, D, generator=g, dtype=dtype),
            torch.randn(B, H, Tk, Dv, generator=g, dtype=dtype))


def test_attention_matches_torch_sdpa():
    q, k, v = _qkv()
    scale = 1 / math.sqrt(q.shape[-1])
    o, _ = O.attention(q, k, v, scale, causal=True)
    torch.testing.assert_close(o, F.scaled_dot_product_attention(q, k, v, is_causal=True), rtol=1e-10, atol=1e-10)
    o2, _ = O.attention(q, k, v, 0.3, causal=False)
    torch.testing.assert_close(o2, F.scaled_dot_product_attention(q, k, v, scale=0.3), rtol=1e-10, atol=1e-10)


def test_attention_matches_bruteforce_loops():
    q, k, v = _qkv(B=1, H=2, Tq=5, Tk=7, D=4, Dv=3, seed=4)
    scale, off = 0.7, 2
    o, lse = O.attention(q, k, v, scale, causal=True, q_offset=off)
    for b in range(1):
        for h in range(2):
            for i in range(5):
                sc = [sum(q[b, h, i, d].item() * k[b, h, j, d].item() for d in range(4)) * scale
                      for j in range(7) if j <= i + off]
                mx = max(sc)
                den = sum(math.exp(s - mx) for s in sc)
                assert abs(lse[b, h, i].item() - (mx + math.log(den))) < 1e-12
                for e in range(3):
                    num = sum(math.exp(s - mx) * v[b, h, j, e].item() for j, s in enumerate(sc))
                    assert abs(o[b, h, i, e].item() - num / den) < 1e-12


def test_attention_mask_equals_reference_triu_construction():
    # transformer.py:273-281 builds triu(full(-inf), diagonal=pos_offset+1) and adds it
    q, k, v = _qkv(Tq=6, Tk=15, seed=5)
    off = 9
    s = q @ k.transpose(-1, -2) * 0.25
    mask = torch.triu(torch.full((6, 15), float("-inf"), dtype=s.dtype), diagonal=off + 1)
    ref = torch.softmax(s + mask, -1) @ v
    o, _ = O.attention(q, k, v, 0.25, causal=True, q_offset=off)
    torch.testing.assert_close(o, ref, rtol=1e-12, atol=1e-12)


def test_attention_invariants():
    q, k, v = _qkv(Tq=33, Tk=33, seed=6)
    scale = 0.2
    o, lse = O.attention(q, k, v, scale)
    # rows of P sum to 1: recompute from lse
    s = (q @ k.transpose(-1, -2)) * scale
    s = s.masked_fill(~torch.ones(33, 33, dtype=torch.bool).tril(), float("-inf"))
    torch.testing.assert_close(torch.exp(s - lse[..., None]).sum(-1), torch.ones_like(lse), rtol=0, atol=1e-12)
    # V = ones  =>  O = 1
    o1, _ = O.attention(q, k, torch.ones_like(v), scale)
    torch.testing.assert_close(o1, torch.ones_like(o1), rtol=0, atol=1e-12)
    # causal: first query sees only key 0
    torch.testing.assert_close(o[..., 0, :], v[..., 0, :], rtol=0, atol=1e-12)
    # prefix independence
    op, _ = O.attention(q[..., :20, :], k[..., :20, :], v[..., :20, :], scale)
    torch.testing.assert_close(op, o[..., :20, :], rtol=1e-12, atol=1e-12)


def test_attention_shared_key_head_broadcast():
    q, k, v = _qkv(H=4, seed=7)
    k1 = k[:, :1]
    o, _ = O.attention(q, k1, v, 0.3)
    o2, _ = O.attention(q, k1.expand_as(k).contiguous(), v, 0.3)
    torch.testing.assert_close(o, o2, rtol=0, atol=0)


# ---------------------------------------------------------------- attention backward

def test_attention_bwd_gradcheck():
    q, k, v = _qkv(B=1, H=1, Tq=6, Tk=6, D=5, Dv=4, seed=8)
    f = lambda q_, k_, v_: O.attention(q_, k_, v_, 0.5, True, 0)[0]
    assert torch.autograd.gradcheck(f, (q.requires_grad_(), k.requires_grad_(), v.requires_grad_()))


def test_attention_bwd_matches_sdpa_autograd():
    q, k, v = _qkv(seed=9)
    do = torch.randn_like(q[..., :16])
    dq, dk, dv = O.attention_bwd(q, k, v, do, 1 / math.sqrt(24), True, 0)
    qq, kk, vv = (t.clone().requires_grad_() for t in (q, k, v))
    F.scaled_dot_product_attention(qq, kk, vv, is_causal=True).backward(do)
    for a, b in ((dq, qq.grad), (dk, kk.grad), (dv, vv.grad)):
        torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-10)


# ---------------------------------------------------------------- absorbed decode

def test_absorbed_decode_equals_expanded_attention():
    g = torch.Generator().manual_seed(10)
    B, H, L, DL, dn, dr, dv = 2, 3, 21, 16, 8, 6, 5
    q_nope = torch.randn(B, H, 1, dn, generator=g, dtype=torch.float64)
    q_rope = torch.randn(B, H, 1, dr, generator=g, dtype=torch.float64)
    c = torch.randn(B, L, DL, generator=g, dtype=torch.float64)
    kr = torch.randn(B, 1, L, dr, generator=g, dtype=torch.float64)
    Wuk = torch.randn(H, dn, DL, generator=g, dtype=torch.float64)
    Wuv = torch.randn(H, dv, DL, generator=g, dtype=torch.float64)
    scale = 0.37
    q_lat = torch.einsum("bhtc,hcd->bhtd", q_nope, Wuk)
    ctx, lse = O.absorbed_decode(q_lat, q_rope, c, kr, scale)
    out = torch.einsum("bhtd,hmd->bhtm", ctx, Wuv)
    k_nope = torch.einsum("bld,hcd->bhlc", c, Wuk)
    v = torch.einsum("bld,hmd->bhlm", c, Wuv)
    q = torch.cat([q_nope, q_rope], -1)
    k = torch.cat([k_nope, kr.expand(B, H, L, dr)], -1)
    ref, ref_lse = O.attention(q, k, v, scale, causal=False)
    torch.testing.assert_close(out, ref, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(lse, ref_lse, rtol=1e-10, atol=1e-10)


def test_absorbed_decode_single_key_and_seq_lens():
    g = torch.Generator().manual_seed(11)
    q_lat = torch.randn(2, 4, 1, 8, generator=g, dtype=torch.float64)
    q_rope = torch.randn(2, 4, 1, 4, generator=g, dtype=torch.float64)
    c = torch.randn(2, 9, 8, generator=g, dtype=torch.float64)
    kr = torch.randn(2, 4, 9, 4, generator=g, dtype=torch.float64)
    ctx, _ = O.absorbed_decode(q_lat, q_rope, c[:, :1], kr[:, :, :1], 0.5)
    torch.testing.assert_close(ctx, c[:, :1].unsqueeze(1).expand(2, 4, 1, 8), rtol=0, atol=1e-14)
    ctx2, lse2 = O.absorbed_decode(q_lat, q_rope, c, kr, 0.5, seq_lens=[3, 9])
    a, la = O.absorbed_decode(q_lat[:1], q_rope[:1], c[:1, :3], kr[:1, :, :3], 0.5)
    torch.testing.assert_close(ctx2[:1], a, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(lse2[:1], la, rtol=1e-12, atol=1e-12)


def test_absorbed_chunk_mask_equals_expanded_and_per_query_prefixes():
    # a chunk of T queries at positions L0 .. L0 + T - 1 over L0 + T keys (transformer.py:273-281)
    g = torch.Generator().manual_seed(13)
    B, H, T, L0, DL, dn, dr, dv = 2, 3, 5, 7, 16, 8, 6, 5
    L = L0 + T
    q_nope = torch.randn(B, H, T, dn, generator=g, dtype=torch.float64)
    q_rope = torch.randn(B, H, T, dr, generator=g, dtype=torch.float64)
    c = torch.randn(B, L, DL, generator=g, dtype=torch.float64)
    kr = torch.randn(B, 1, L, dr, generator=g, dtype=torch.float64)
    Wuk = torch.randn(H, dn, DL, generator=g, dtype=torch.float64)
    Wuv = torch.randn(H, dv, DL, generator=g, dtype=torch.float64)
    q_lat = torch.einsum("bhtc,hcd->bhtd", q_nope, Wuk)
    ctx, lse = O.absorbed_decode(q_lat, q_rope, c, kr, 0.41, q_offset=L0)
    # expanded form: K = [c W_UK^T, k_rope], V = c W_UV^T under SDPA's bottom-right offset
    k = torch.cat([torch.einsum("bld,hcd->bhlc", c, Wuk), kr.expand(B, H, L, dr)], -1)
    v = torch.einsum("bld,hmd->bhlm", c, Wuv)
    ref, ref_lse = O.attention(torch.cat([q_nope, q_rope], -1), k, v, 0.41, causal=True, q_offset=L0)
    torch.testing.assert_close(torch.einsum("bhtd,hmd->bhtm", ctx, Wuv), ref, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(lse, ref_lse, rtol=1e-10, atol=1e-10)
    # query t alone over the prefix of L0 + t + 1 keys
    for t in range(T):
        a, la = O.absorbed_decode(q_lat[:, :, t:t + 1], q_rope[:, :, t:t + 1], c[:, :L0 + t + 1],
                                  kr[:, :, :L0 + t + 1], 0.41)
        torch.testing.assert_close(ctx[:, :, t:t + 1], a, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(lse[:, :, t:t + 1], la, rtol=1e-12, atol=1e-12)
    # the reference's own additive mask construction gives the same scores' softmax
    s = (q_lat @ c.unsqueeze(1).transpose(-1, -2) + q_rope @ kr.transpose(-1, -2)) * 0.41
    s = s + torch.triu(torch.full((T, L), float("-inf"), dtype=torch.float64), diagonal=L0 + 1)
    torch.testing.assert_close(torch.softmax(s, -1) @ c.unsqueeze(1), ctx, rtol=1e-12, atol=1e-12)


def test_split_merge_equals_full_softmax():
    g = torch.Generator().manual_seed(12)
    q_lat = torch.randn(1, 2, 1, 8, generator=g, dtype=torch.float64)
    q_rope = torch.randn(1, 2, 1, 4, generator=g, dtype=torch.float64)
    c = torch.randn(1, 30, 8, generator=g, dtype=torch.float64)
    kr = torch.randn(1, 1, 30, 4, generator=g, dtype=torch.float64)
    full, lse = O.absorbed_decode(q_lat, q_rope, c, kr, 0.8)
    parts = [O.absorbed_decode(q_lat, q_rope, c[:, a:b], kr[:, :, a:b], 0.8) for a, b in ((0, 7), (7, 19), (19, 30))]
    m, ml = O.merge_splits(torch.stack([p[0] for p in parts]), torch.stack([p[1] for p in parts]))
    torch.testing.assert_close(m, full, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(ml, lse, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- whole module vs reference vectors

def _w(golden):
    return {k: v.double() for k, v in golden.weights.items()}


def test_mla_train_branch_matches_reference_golden(golden):
    dims = golden.dims
    w = {k: v.clone().requires_grad_(True) for k, v in _w(golden).items()}
    x = golden.t("train.x").double().requires_grad_(True)
    y, cache = O.mla_forward(w, x, dims)
    assert cache is None
    torch.testing.assert_close(y.float(), golden.t("train.y"), rtol=0, atol=2e-6)
    y.backward(golden.t("train.dy").double())
    torch.testing.assert_close(x.grad.float(), golden.t("train.dx"), rtol=0, atol=2e-6)
    torch.testing.assert_close(w["k_up.weight"].grad.float(), golden.t("train.dk_up"), rtol=0, atol=2e-6)


def test_mla_cache_branch_matches_reference_golden(golden):
    dims, w = golden.dims, _w(golden)
    y, c = O.mla_forward(w, golden.t("prefill.x"), dims, None, True)
    torch.testing.assert_close(y.float(), golden.t("prefill.y"), rtol=0, atol=2e-6)
    torch.testing.assert_close(c["latent"].float(), golden.t("prefill.latent"), rtol=0, atol=2e-6)
    torch.testing.assert_close(c["k_rope"].float(), golden.t("prefill.k_rope"), rtol=0, atol=2e-6)
    assert c["seq_len"] == int(golden.raw["prefill.seq_len"])
    for i in range(3):
        y, c = O.mla_forward(w, golden.t(f"decode{i}.x"), dims, c, True)
        torch.testing.assert_close(y.float(), golden.t(f"decode{i}.y"), rtol=0, atol=2e-6)
    y, c = O.mla_forward(w, golden.t("chunk.x"), dims, c, True)
    torch.testing.assert_close(y.float(), golden.t("chunk.y"), rtol=0, atol=2e-6)
    torch.testing.assert_close(c["latent"].float(), golden.t("chunk.latent"), rtol=0, atol=2e-6)
    torch.testing.assert_close(c["k_rope"].float(), golden.t("chunk.k_rope"), rtol=0, atol=2e-6)
    assert c["seq_len"] == int(golden.raw["chunk.seq_len"])


@pytest.mark.parametrize("shared", [False, True])
def test_mla_cache_decode_equals_no_cache_forward(shared):
    # decode-after-prefill on the concatenated sequence == the no-cache forward
    dims = O.MLADims(d_model=48, n_heads=3, q_lora_rank=32, d_latent=32, qk_nope_dim=16, qk_rope_dim=64,
                     v_head_dim=24, n_k_rope_heads=1 if shared else 3, max_seq_len=64)
    g = torch.Generator().manual_seed(13)
    w = O.init_weights(dims, g, std=0.1, dtype=torch.float64)
    x = torch.randn(2, 11, 48, generator=g, dtype=torch.float64)
    full, _ = O.mla_forward(w, x, dims)
    y0, c = O.mla_forward(w, x[:, :7], dims, None, True)
    parts = [y0]
    for t in range(7, 9):
        y, c = O.mla_forward(w, x[:, t:t + 1], dims, c, True)
        parts.append(y)
    y, c = O.mla_forward(w, x[:, 9:], dims, c, True)
    parts.append(y)
    torch.testing.assert_close(torch.cat(parts, 1), full, rtol=1e-10, atol=1e-10)


def test_robust_diff_reporting():
    a = torch.zeros(1000)
    b = torch.zeros(1000)
    b[0] = 1.0
    m = O.robust_diff(a, b)
    assert m["max"] == 1.0 and abs(m["mean"] - 1e-3) < 1e-12 and m["p99"] == 0.0


# ---------------------------------------------------------------- RMSNorm (norm1 -> down-projections)

def test_rms_norm_matches_library_rms_norm():
    g = torch.Generator().manual_seed(21)
    x = torch.randn(5, 7, 96, generator=g, dtype=torch.float64)
    w = torch.randn(96, generator=g, dtype=torch.float64)
    for eps in (1e-6, 0.3):
        ref = F.rms_norm(x, (96,), w, eps)
        torch.testing.assert_close(O.rms_norm(x, w, eps), ref, rtol=1e-13, atol=1e-13)


def test_rms_norm_closed_forms():
    w = torch.linspace(-2, 3, 16, dtype=torch.float64)
    # a constant row c: mean(x^2) = c^2, so y = c / sqrt(c^2 + eps) * w
    for c, eps in ((3.0, 0.0), (-0.5, 1e-6), (2.0, 4.0)):
        y = O.rms_norm(torch.full((1, 16), c, dtype=torch.float64), w, eps)
        torch.testing.assert_close(y[0], c / math.sqrt(c * c + eps) * w, rtol=1e-14, atol=1e-14)
    g = torch.Generator().manual_seed(22)
    x = torch.randn(9, 40, generator=g, dtype=torch.float64)
    # eps = 0: every row of y / w has mean square 1, and the norm ignores the row's scale
    y = O.rms_norm(x, None, 0.0)
    torch.testing.assert_close(y.pow(2).mean(-1), torch.ones(9, dtype=torch.float64), rtol=1e-13, atol=1e-13)
    torch.testing.assert_close(O.rms_norm(7.5 * x, None, 0.0), y, rtol=1e-13, atol=1e-13)


def test_rms_norm_bwd_gradcheck_and_scale_invariance():
    g = torch.Generator().manual_seed(23)
    x = torch.randn(3, 24, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(24, generator=g, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda a, b: O.rms_norm(a, b, 1e-3), (x, w))
    dy = torch.randn(3, 24, generator=g, dtype=torch.float64)
    dx, dw = O.rms_norm_bwd(x.detach(), w.detach(), dy, eps=0.0)
    # a row-scale-invariant map has a gradient orthogonal to its input row
    torch.testing.assert_close((dx * x.detach()).sum(-1), torch.zeros(3, dtype=torch.float64), rtol=0, atol=1e-12)
    # dw = sum over rows of dy * x r
    r = x.detach().pow(2).mean(-1, keepdim=True).rsqrt()
    torch.testing.assert_close(dw, (dy * x.detach() * r).sum(0), rtol=1e-13, atol=1e-13)


def test_rmsnorm_down_proj_identity_and_exact_rows():
    g = torch.Generator().manual_seed(24)
    K = 64
    x = torch.randn(6, K, generator=g).to(torch.bfloat16)
    w_norm = torch.randn(K, generator=g).to(torch.bfloat16)
    # identity w_down: the bf16-rounded norm itself (the reference's own division form)
    eye = torch.eye(K, dtype=torch.bfloat16)
    y = O.rmsnorm_down_proj(x, w_norm, eye, 1e-6)
    xf = x.float()
    xn = (xf / torch.sqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * w_norm.float()).to(torch.bfloat16)
    assert torch.equal(y, xn)
    # the reference kernel's rsqrt form agrees with the division form within one bf16 ulp
    alt = O.rms_norm(xf, w_norm.float(), 1e-6).to(torch.bfloat16)
    assert ((alt.float() - xn.float()).abs() <= xn.float().abs() * 2 ** -8 + 1e-30).all()
    # rows of equal magnitude: r = 1 / |c| at eps = 0, so y = sign * w_norm @ w_down exactly
    signs = torch.tensor([1.0, -1.0] * (K // 2))
    xr = (signs * 4.0).to(torch.bfloat16)[None]
    w_down = torch.randint(-3, 4, (K, 8), generator=g).to(torch.bfloat16)
    w1 = torch.ones(K, dtype=torch.bfloat16)
    y = O.rmsnorm_down_proj(xr, w1, w_down, 0.0)
    assert torch.equal(y.float(), (signs[None] @ w_down.float()))


# ---------------------------------------------------------------- vocabulary-chunked linear cross-entropy

@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_chunked_ce_matches_library_cross_entropy(reduction):
    g = torch.Generator().manual_seed(31)
    x = torch.randn(2, 7, 24, generator=g, dtype=torch.float64)
    w = torch.randn(100, 24, generator=g, dtype=torch.float64) * 0.5
    y = torch.randint(0, 100, (2, 7), generator=g)
    ref = F.cross_entropy((x.reshape(14, 24) @ w.t()), y.reshape(14), reduction=reduction)
    for chunk in (8, 37, 64, 100, 4096):
        got = O.chunked_linear_cross_entropy(x, w, y, chunk, reduction)
        torch.testing.assert_close(got.reshape(ref.shape), ref, rtol=1e-12, atol=1e-12)


def test_chunked_ce_closed_form_and_gradcheck():
    # zero weights: every logit is 0, so each loss is log V
    x = torch.randn(1, 5, 16, dtype=torch.float64)
    loss = O.chunked_linear_cross_entropy(x, torch.zeros(40, 16, dtype=torch.float64),
                                          torch.arange(5).view(1, 5), 16, "none")
    torch.testing.assert_close(loss, torch.full((1, 5), math.log(40), dtype=torch.float64), rtol=1e-14, atol=1e-14)
    g = torch.Generator().manual_seed(32)
    xx = torch.randn(1, 3, 8, generator=g, dtype=torch.float64, requires_grad=True)
    ww = torch.randn(24, 8, generator=g, dtype=torch.float64, requires_grad=True)
    y = torch.tensor([[0, 23, 9]])
    assert torch.autograd.gradcheck(lambda a, b: O.chunked_linear_cross_entropy(a, b, y, 8, "mean"), (xx, ww))
