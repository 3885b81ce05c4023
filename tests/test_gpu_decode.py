"""GPU parity of the absorbed latent decode (mla_decode) against the oracle's
absorbed_decode (transformer.py:249-286, T == 1).

Tolerance: ctx (bf16) within max-abs 2e-2 / mean-abs 2e-3 of the fp64 oracle on
the same bf16 inputs; LSE within 1e-3.
"""
import math

import pytest
import torch

from oracle import mla_oracle as O
from tests.gpu_util import check_close, randn_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import transformer_amd  # noqa: F401
    return torch.ops.mla_mi355x


def make(B, H, L, DL, Hr, seed, q_scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (randn_bf16((B, H, DL), g, q_scale), randn_bf16((B, H, 64), g, q_scale),
            randn_bf16((B, L, DL), g), randn_bf16((B, Hr, L, 64), g))


def oracle(q_lat, q_rope, c, kr, scale, seq_lens=None):
    ctx, lse = O.absorbed_decode(q_lat.double().unsqueeze(2), q_rope.double().unsqueeze(2), c.double(),
                                 kr.double(), scale, seq_lens)
    return ctx.squeeze(2), lse.squeeze(2)


def run(ops, q_lat, q_rope, c, kr, scale, seq_lens=None, splits=0):
    sl = None if seq_lens is None else torch.tensor(seq_lens, dtype=torch.int32).cuda()
    ctx, lse = ops.decode(q_lat.cuda(), q_rope.cuda(), c.cuda(), kr.cuda(), sl, scale, splits)
    torch.cuda.synchronize()
    return ctx.cpu(), lse.cpu()


CASES = [
    # B, H, L, DL, Hr, splits
    (1, 1, 1, 64, 1, 0),
    (2, 16, 64, 512, 1, 0),
    (3, 16, 777, 512, 1, 0),
    (2, 14, 300, 384, 14, 0),   # reference layout: per-head k_rope, H = 14, d_latent 384
    (2, 4, 129, 64, 4, 2),
    (1, 20, 500, 256, 1, 3),    # two head groups, the second partial
    (4, 16, 1000, 128, 1, 1),   # single split: direct write path
    (2, 16, 4096, 512, 1, 64),  # many splits
    (3, 16, 3000, 512, 1, 0),   # 23 automatic splits: the merge walks three chunks of 8
    (1, 16, 20000, 512, 1, 0),  # one sequence: 156 automatic splits, the wide merge
    (1, 16, 20000, 512, 1, 400),  # 313 splits: merge groups take two chunks of 8
    (1, 20, 9000, 256, 1, 0),   # wide merge over two head groups, the second partial
]


@pytest.mark.parametrize("B,H,L,DL,Hr,splits", CASES)
def test_decode_matches_oracle(ops, B, H, L, DL, Hr, splits):
    print(f"case B={B} H={H} L={L} DL={DL} Hr={Hr} splits={splits}", flush=True)
    q_lat, q_rope, c, kr = make(B, H, L, DL, Hr, seed=L + DL)
    scale = 1 / math.sqrt(192)
    ctx, lse = run(ops, q_lat, q_rope, c, kr, scale, splits=splits)
    rc, rl = oracle(q_lat, q_rope, c, kr, scale)
    check_close(ctx.double(), rc, "ctx")
    torch.testing.assert_close(lse.double(), rl, rtol=0, atol=1e-3)


def test_decode_config2_shape(ops):
    # the benchmark decode shape: batch 32, context 4096, c_kv[512] + shared k_rope[64], 16 heads
    q_lat, q_rope, c, kr = make(32, 16, 4096, 512, 1, seed=2)
    scale = 1 / math.sqrt(192)
    ctx, lse = run(ops, q_lat, q_rope, c, kr, scale)
    rc, rl = oracle(q_lat, q_rope, c, kr, scale)
    check_close(ctx.double(), rc, "ctx (config 2)")
    torch.testing.assert_close(lse.double(), rl, rtol=0, atol=1e-3)


def test_decode_peaked(ops):
    q_lat, q_rope, c, kr = make(2, 16, 1024, 512, 1, seed=3, q_scale=4.0)
    scale = 1 / math.sqrt(192)
    ctx, lse = run(ops, q_lat, q_rope, c, kr, scale)
    rc, rl = oracle(q_lat, q_rope, c, kr, scale)
    check_close(ctx.double(), rc, "ctx (peaked)")
    torch.testing.assert_close(lse.double(), rl, rtol=0, atol=1e-3)


def test_decode_seq_lens_ragged_and_empty(ops):
    B, H, L, DL = 5, 16, 700, 512
    q_lat, q_rope, c, kr = make(B, H, L, DL, 1, seed=4)
    lens = [1, 700, 0, 333, 64]
    scale = 0.07
    ctx, lse = run(ops, q_lat, q_rope, c, kr, scale, seq_lens=lens)
    for b, n in enumerate(lens):
        if n == 0:
            assert (ctx[b] == 0).all() and torch.isinf(lse[b]).all() and (lse[b] < 0).all()
            continue
        rc, rl = oracle(q_lat[b:b + 1], q_rope[b:b + 1], c[b:b + 1, :n], kr[b:b + 1, :, :n], scale)
        check_close(ctx[b:b + 1].double(), rc, f"ctx (b={b}, len={n})")
        torch.testing.assert_close(lse[b:b + 1].double(), rl, rtol=0, atol=1e-3)
    # length 1: ctx is exactly c_kv[0] (up to bf16 rounding of a weight-1 average)
    assert (ctx[0].float() - c[0, 0].float()).abs().max().item() <= 1e-2


def test_decode_seq_lens_far_below_capacity(ops):
    # a capacity-sized cache with short lengths: each sequence's length is split at run time
    B, H, L, DL = 4, 16, 4096, 512
    q_lat, q_rope, c, kr = make(B, H, L, DL, 1, seed=5)
    lens = [100, 4096, 2500, 1]
    scale = 0.05
    ctx, lse = run(ops, q_lat, q_rope, c, kr, scale, seq_lens=lens, splits=8)
    for b, n in enumerate(lens):
        rc, rl = oracle(q_lat[b:b + 1], q_rope[b:b + 1], c[b:b + 1, :n], kr[b:b + 1, :, :n], scale)
        check_close(ctx[b:b + 1].double(), rc, f"ctx (b={b}, len={n})")
        torch.testing.assert_close(lse[b:b + 1].double(), rl, rtol=0, atol=1e-3)


@pytest.mark.parametrize("DL,Hr", [(512, 1), (128, 16)])
def test_decode_seq_lens_ignore_rows_past_the_length(ops, DL, Hr):
    # positions past a sequence's length in a capacity-sized cache may hold anything (a grown
    # buffer is not cleared): filled with NaN, the result must equal the zero-filled one
    # (regression: a tile's rows past the length were read, and p = 0 met NaN in the PV product)
    B, H, L = 3, 16, 700
    q_lat, q_rope, c, kr = make(B, H, L, DL, Hr, seed=12)
    lens = [515, 1, 690]
    cz, kz, cn, kn = c.clone(), kr.clone(), c.clone(), kr.clone()
    for b, n in enumerate(lens):
        cz[b, n:] = 0
        kz[b, :, n:] = 0
        cn[b, n:] = float("nan")
        kn[b, :, n:] = float("nan")
    for splits in (0, 1, 5):
        print(f"case DL={DL} Hr={Hr} splits={splits}", flush=True)
        ctx_z, lse_z = run(ops, q_lat, q_rope, cz, kz, 0.05, seq_lens=lens, splits=splits)
        ctx_n, lse_n = run(ops, q_lat, q_rope, cn, kn, 0.05, seq_lens=lens, splits=splits)
        assert torch.isfinite(ctx_n.float()).all() and torch.isfinite(lse_n).all()
        assert torch.equal(ctx_n, ctx_z) and torch.equal(lse_n, lse_z)


def test_decode_strided_cache_views(ops):
    # latent cache as a prefix view of a preallocated [B, Lmax, DL] buffer, k_rope as a
    # view of [B, 1, Lmax, 64]; query heads as views of wider projections
    g = torch.Generator().manual_seed(5)
    B, H, L, Lmax, DL = 3, 16, 450, 1024, 512
    cbuf = randn_bf16((B, Lmax, DL), g).cuda()
    kbuf = randn_bf16((B, 1, Lmax, 64), g).cuda()
    qbuf = randn_bf16((B, H, DL + 64), g).cuda()
    c, kr = cbuf[:, :L], kbuf[:, :, :L]
    q_lat, q_rope = qbuf[..., :DL], qbuf[..., DL:]
    ctx, lse = ops.decode(q_lat, q_rope, c, kr, None, 0.1, 0)
    rc, rl = oracle(q_lat.cpu(), q_rope.cpu(), c.cpu(), kr.cpu(), 0.1)
    check_close(ctx.cpu().double(), rc, "ctx (strided)")


def test_decode_split_count_invariance_and_determinism(ops):
    q_lat, q_rope, c, kr = (t.cuda() for t in make(2, 16, 2048, 512, 1, seed=6))
    outs = [ops.decode(q_lat, q_rope, c, kr, None, 0.1, s) for s in (1, 4, 16, 64)]
    for ctx, lse in outs[1:]:
        assert (ctx.float() - outs[0][0].float()).abs().max().item() <= 1e-2
        torch.testing.assert_close(lse, outs[0][1], rtol=0, atol=1e-4)
    again = ops.decode(q_lat, q_rope, c, kr, None, 0.1, 4)
    assert torch.equal(again[0], outs[1][0]) and torch.equal(again[1], outs[1][1])
    again = ops.decode(q_lat, q_rope, c, kr, None, 0.1, 16)  # two 8-split chunks per merge thread
    assert torch.equal(again[0], outs[2][0]) and torch.equal(again[1], outs[2][1])
    again = ops.decode(q_lat, q_rope, c, kr, None, 0.1, 64)  # the wide merge
    assert torch.equal(again[0], outs[3][0]) and torch.equal(again[1], outs[3][1])


def test_decode_rejects_bad_inputs(ops):
    q_lat, q_rope, c, kr = (t.cuda() for t in make(1, 4, 16, 512, 1, seed=7))
    with pytest.raises(ValueError):
        ops.decode(q_lat[..., :500].contiguous(), q_rope, c[..., :500].contiguous(), kr, None, 0.1, 0)
    with pytest.raises(ValueError):
        ops.decode(q_lat, q_rope, c, kr.expand(1, 2, 16, 64), None, 0.1, 0)


# ---------------------------------------------------------------- decode with the W_UV product fused

OUT_CASES = [
    # B, H, L, DL, Hr, splits, seq_lens
    (1, 1, 1, 64, 1, 0, None),
    (5, 16, 777, 512, 1, 0, None),        # B not a multiple of the 4 sequences per merge workgroup
    (2, 14, 300, 384, 14, 0, None),       # reference layout
    (3, 20, 500, 256, 1, 3, None),        # two head groups
    (4, 16, 1000, 128, 1, 1, None),       # single split: ctx goes through the workspace scratch
    (6, 16, 640, 512, 1, 0, [640, 0, 1, 17, 639, 300]),  # ragged and empty sequences
    (32, 16, 4096, 512, 1, 0, None),      # config 2
    (1, 16, 1536, 512, 1, 0, [1000]),     # 12 splits over the capacity, 8 used: the W_UV merge walks 2 chunks
    (2, 16, 4096, 512, 1, 0, [4096, 2500]),  # 32 splits, ragged: the W_UV merge walks 4 chunks
    (1, 16, 20000, 512, 1, 0, None),      # wide merge, then W_UV from the workspace's ctx scratch
    (2, 20, 9000, 256, 1, 0, [9000, 5000]),  # wide merge over two head groups, ragged
]


@pytest.mark.parametrize("B,H,L,DL,Hr,splits,seq_lens", OUT_CASES)
def test_decode_out_matches_oracle_and_unfused(ops, B, H, L, DL, Hr, splits, seq_lens):
    print(f"case B={B} H={H} L={L} DL={DL} Hr={Hr} splits={splits} seq_lens={seq_lens}", flush=True)
    q_lat, q_rope, c, kr = make(B, H, L, DL, Hr, seed=3 * L + DL)
    g = torch.Generator().manual_seed(B + H)
    w_uv = randn_bf16((H, 128, DL), g, 0.05)  # v_up.weight.view(H, d_v, DL)
    scale = 1 / math.sqrt(192)
    sl = None if seq_lens is None else torch.tensor(seq_lens, dtype=torch.int32).cuda()
    out, lse = ops.decode_out(q_lat.cuda(), q_rope.cuda(), c.cuda(), kr.cuda(), sl, w_uv.cuda(), scale, splits)
    assert out.shape == (B, H, 128) and out.is_contiguous()
    # the oracle: fp64 absorbed decode, then ctx W_UV^T per head (transformer.py:286-291)
    ctx_ref, lse_ref = oracle(q_lat, q_rope, c, kr, scale, seq_lens)
    if seq_lens is not None:  # an empty sequence has no softmax; the kernel's contract is ctx = 0
        ctx_ref[torch.tensor(seq_lens) == 0] = 0.0
    out_ref = torch.einsum("bhc,hdc->bhd", ctx_ref, w_uv.double())
    check_close(out.float(), out_ref, "out")
    fin = torch.isfinite(lse_ref)
    assert torch.equal(torch.isfinite(lse.cpu()), fin)
    torch.testing.assert_close(lse.cpu().double()[fin], lse_ref[fin], rtol=0, atol=1e-3)
    if seq_lens is not None:
        for i, n in enumerate(seq_lens):
            if n == 0:
                assert (out[i] == 0).all(), "an empty sequence must give out = 0"
    # against the unfused path: the same bf16 ctx times W_UV in fp32, one rounding
    ctx, lse2 = ops.decode(q_lat.cuda(), q_rope.cuda(), c.cuda(), kr.cuda(), sl, scale, splits)
    assert torch.equal(lse2, lse)
    unf = torch.einsum("bhc,hdc->bhd", ctx.double().cpu(), w_uv.double())
    e = unf.abs().clamp_min(2.0 ** -20)
    assert ((out.cpu().double() - unf).abs() <= e * 2.0 ** -8 + 1e-6).all(), "beyond one bf16 ulp of the unfused path"
    again, _ = ops.decode_out(q_lat.cuda(), q_rope.cuda(), c.cuda(), kr.cuda(), sl, w_uv.cuda(), scale, splits)
    assert torch.equal(again, out), "decode_out is not bitwise reproducible"


def test_decode_out_rejects_bad_weights(ops):
    q_lat, q_rope, c, kr = make(2, 4, 32, 64, 1, seed=1)
    with pytest.raises(ValueError):
        ops.decode_out(q_lat.cuda(), q_rope.cuda(), c.cuda(), kr.cuda(), None,
                       torch.zeros(4, 96, 64, dtype=torch.bfloat16, device="cuda"), 0.1, 0)  # d_v 96


@pytest.mark.parametrize("B,H,dn,DL", [(1, 1, 128, 512), (5, 16, 128, 512), (2, 14, 64, 384), (3, 4, 128, 64),
                                       (32, 16, 128, 512)])
def test_absorb_q_matches_oracle(ops, B, H, dn, DL):
    # q_lat = q_nope W_UK per head (transformer.py:252-254); q_nope read as a strided view of q_up's rows
    g = torch.Generator().manual_seed(B * 7 + DL)
    rows = randn_bf16((B, 1, H * dn + 64), g)  # a wider row: the q view is strided
    w_uk = randn_bf16((H, dn, DL), g, 0.05)
    q = rows.cuda()[:, 0, :H * dn].view(B, H, dn)
    q_lat = ops.absorb_q(q, w_uk.cuda())
    ref = torch.einsum("bhd,hdc->bhc", rows[:, 0, :H * dn].view(B, H, dn).double(), w_uk.double())
    assert q_lat.shape == (B, H, DL)
    check_close(q_lat.float(), ref, "q_lat", max_abs=2e-2 * max(1.0, ref.abs().max().item()))
    e = ref.abs().clamp_min(2.0 ** -20)
    assert ((q_lat.cpu().double() - ref).abs() <= e * 2.0 ** -8 + 1e-5).all(), "beyond one bf16 ulp of fp64"
    assert torch.equal(ops.absorb_q(q, w_uk.cuda()), q_lat)


@pytest.mark.parametrize("B,L,splits", [(4, 1000, 1), (8, 2048, 0), (1, 20000, 0)])
def test_decode_out_writes_a_caller_ctx(ops, B, L, splits):
    # mla_decode_out with the caller's ctx (through the C-ABI; the op passes none): one split
    # (the main kernel writes ctx), up to 32 (16 here: the W_UV merge writes it) and more than 32
    # (the wide merge writes it and the W_UV product reads it back).  Every output equals the op's
    # and mla_decode's bit for bit.
    import ctypes
    from transformer_amd import _lib, kernels
    H, DL = 16, 512
    print(f"case decode_out with a caller ctx B={B} L={L} splits={splits}", flush=True)
    q_lat, q_rope, c, kr = (t.cuda() for t in make(B, H, L, DL, 1, seed=L + 7))
    g = torch.Generator().manual_seed(9)
    w_uv = (torch.randn(H, 128, DL, generator=g) * 0.05).to(torch.bfloat16).cuda()
    scale = 1 / math.sqrt(192)
    out_ref, lse_ref = ops.decode_out(q_lat, q_rope, c, kr, None, w_uv, scale, splits)
    ctx_ref, lse_dec = ops.decode(q_lat, q_rope, c, kr, None, scale, splits)
    ctx = torch.full((B, H, DL), float("nan"), dtype=torch.bfloat16, device="cuda")
    lse = torch.full((B, H), float("nan"), device="cuda")
    out = torch.full((B, H, 128), float("nan"), dtype=torch.bfloat16, device="cuda")
    dargs, keep = kernels._decode_args("mla_decode_out", q_lat, q_rope, c, kr, None, scale, splits, ctx, lse)
    args = _lib.DecodeOutArgs(dec=dargs, w_uv=w_uv.data_ptr(), out=out.data_ptr(), w_uv_sh=w_uv.stride(0),
                              w_uv_sd=w_uv.stride(1), out_sb=out.stride(0), out_sh=out.stride(1), d_v=128)
    n = int(_lib.entry("mla_decode_out_workspace_bytes")(ctypes.byref(args)))
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device="cuda")
    args.dec.workspace, args.dec.workspace_bytes = ws.data_ptr(), n
    _lib.check(_lib.entry("mla_decode_out")(ctypes.byref(args), torch.cuda.current_stream().cuda_stream),
               "mla_decode_out")
    torch.cuda.synchronize()
    assert torch.equal(out, out_ref) and torch.equal(lse, lse_ref), "out / lse differ from the op's"
    assert torch.equal(ctx, ctx_ref) and torch.equal(lse, lse_dec), "ctx / lse differ from mla_decode's"
