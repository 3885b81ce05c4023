"""GPU parity of the absorbed prefill with a cache (mla_prefill_cached) against the oracle's
absorbed_decode with the chunk mask (transformer.py:247-286 for T > 1: query t of the chunk
at position L0 + t sees keys 0 .. L0 + t, the mask triu(diagonal=pos_offset+1) of :273-281).

Tolerance: ctx (bf16) within max-abs 2e-2 / mean-abs 2e-3 of the fp64 oracle on the same
bf16 inputs; LSE within 1e-3 (absolute, natural log)."""
import math

import pytest
import torch

from oracle import mla_oracle as O
from tests.gpu_util import check_close, randn_bf16

pytestmark = pytest.mark.gpu

SCALE = 1 / math.sqrt(192)


@pytest.fixture(scope="module")
def ops():
    import transformer_amd  # noqa: F401
    return torch.ops.mla_mi355x


def make(B, T, H, L, DL, seed, q_scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (randn_bf16((B, T, H, DL), g, q_scale), randn_bf16((B, T, H, 64), g, q_scale),
            randn_bf16((B, L, DL), g), randn_bf16((B, 1, L, 64), g))


def oracle(q_lat, q_rope, c, kr, L0, T):
    """fp64 oracle over the L0 + T rows the chunk sees; [B, T, H, DL] and [B, H, T]."""
    n = L0 + T
    ctx, lse = O.absorbed_decode(q_lat.double().transpose(1, 2), q_rope.double().transpose(1, 2),
                                 c[:, :n].double(), kr[:, :, :n].double(), SCALE, q_offset=L0)
    return ctx.transpose(1, 2), lse


def run(ops, q_lat, q_rope, c, kr, L0):
    ctx, lse = ops.prefill_cached(q_lat.cuda(), q_rope.cuda(), c.cuda(), kr.cuda(), L0, SCALE)
    torch.cuda.synchronize()
    return ctx.cpu(), lse.cpu()


CASES = [
    # B, T, H, L0, spare rows past L0 + T, DL
    (1, 1, 1, 0, 0, 128),        # one query, one key
    (2, 7, 20, 5, 3, 512),       # T not a multiple of the query block; a partial second head group
    (2, 64, 16, 300, 5, 512),    # a chunk over a short cache
    (1, 33, 16, 0, 0, 256),      # no past: the chunk is a whole prompt
    (3, 16, 16, 1000, 16, 384),
    (2, 40, 3, 61, 0, 128),      # 3 heads of a 16-head group
]


@pytest.mark.parametrize("B,T,H,L0,spare,DL", CASES)
def test_prefill_cached_matches_oracle(ops, B, T, H, L0, spare, DL):
    print(f"case B={B} T={T} H={H} L0={L0} spare={spare} DL={DL}", flush=True)
    L = L0 + T + spare
    q_lat, q_rope, c, kr = make(B, T, H, L, DL, seed=T * 7 + L0 + DL)
    if spare:  # rows past the chunk are never read: NaN there must not reach the result
        c[:, L0 + T:] = float("nan")
        kr[:, :, L0 + T:] = float("nan")
    ctx, lse = run(ops, q_lat, q_rope, c, kr, L0)
    assert ctx.shape == (B, T, H, DL) and lse.shape == (B, H, T)
    rc, rl = oracle(q_lat, q_rope, c, kr, L0, T)
    check_close(ctx.double(), rc, "ctx")
    torch.testing.assert_close(lse.double(), rl, rtol=0, atol=1e-3)


@pytest.mark.parametrize("B,T,H,L0,DL", [(32, 64, 16, 150, 512), (40, 50, 20, 77, 384)])
def test_prefill_cached_eight_wave_workgroups(ops, B, T, H, L0, DL):
    # grids of at least 256 eight-query workgroups take the 8-wave kernel (smaller ones the
    # 4-wave kernel, as in the cases above); a partial last query block and head group here
    print(f"case 8-wave B={B} T={T} H={H} L0={L0} DL={DL}", flush=True)
    q_lat, q_rope, c, kr = make(B, T, H, L0 + T, DL, seed=B + T + DL)
    ctx, lse = run(ops, q_lat, q_rope, c, kr, L0)
    rc, rl = oracle(q_lat, q_rope, c, kr, L0, T)
    check_close(ctx.double(), rc, "ctx (8-wave)")
    torch.testing.assert_close(lse.double(), rl, rtol=0, atol=1e-3)


def test_prefill_cached_benchmark_sequence(ops):
    # one sequence of the benchmark chunk (L0 = 4000 cached tokens, a 64-token chunk, 16 heads,
    # c_kv[512] + shared k_rope[64]); the other sequence runs the same code
    print("case benchmark sequence", flush=True)
    B, T, H, L0, DL = 2, 64, 16, 4000, 512
    q_lat, q_rope, c, kr = make(B, T, H, L0 + T, DL, seed=4)
    ctx, lse = run(ops, q_lat, q_rope, c, kr, L0)
    rc, rl = oracle(q_lat[:1], q_rope[:1], c[:1], kr[:1], L0, T)
    check_close(ctx[:1].double(), rc, "ctx (benchmark sequence)")
    torch.testing.assert_close(lse[:1].double(), rl, rtol=0, atol=1e-3)
    # the second sequence: each of its queries' context is a convex combination of cache rows
    assert torch.isfinite(ctx[1].float()).all()


def test_prefill_cached_peaked_and_strided(ops):
    # large scores (the running max moves often) and inputs read through strided views
    print("case peaked + strided", flush=True)
    B, T, H, L0, DL = 2, 24, 16, 200, 512
    g = torch.Generator().manual_seed(9)
    qbuf = randn_bf16((B, T, H, DL + 64 + 8), g, 4.0)  # q_lat and q_rope as views of one buffer
    q_lat, q_rope = qbuf[..., :DL], qbuf[..., DL + 8:]
    cbuf = randn_bf16((B, L0 + T, DL + 64), g)  # c_kv and k_rope as views of one cache row
    c = cbuf[..., :DL]
    kr = cbuf[..., DL:].unsqueeze(1)
    ctx, lse = ops.prefill_cached(q_lat.cuda(), q_rope.cuda(), c.cuda(), kr.cuda(), L0, SCALE)
    rc, rl = oracle(q_lat, q_rope, c, kr, L0, T)
    check_close(ctx.cpu().double(), rc, "ctx (peaked, strided)")
    torch.testing.assert_close(lse.cpu().double(), rl, rtol=0, atol=1e-3)


def test_prefill_cached_t1_equals_decode(ops):
    # T = 1 is the decode step: the same keys, the same softmax
    print("case T=1 vs decode", flush=True)
    B, H, L, DL = 3, 16, 517, 512
    q_lat, q_rope, c, kr = make(B, 1, H, L, DL, seed=5)
    ctx, lse = run(ops, q_lat, q_rope, c, kr, L - 1)
    d_ctx, d_lse = ops.decode(q_lat[:, 0].cuda(), q_rope[:, 0].cuda(), c.cuda(), kr.cuda(), None, SCALE, 1)
    check_close(ctx[:, 0].double(), d_ctx.cpu().double(), "T=1 vs decode", max_abs=1.6e-2, mean_abs=1e-3)
    torch.testing.assert_close(lse[:, :, 0], d_lse.cpu(), rtol=0, atol=1e-4)


def test_prefill_cached_key_ranges(ops):
    # one sequence's chunk leaves most of the chip idle, so the keys are split into ranges whose
    # partials a second kernel merges: every split count gives the oracle's result, and counts
    # that cut the ranges alike give the same bits
    print("case key ranges", flush=True)
    B, T, H, L0, DL = 1, 40, 16, 1500, 512
    q_lat, q_rope, c, kr = make(B, T, H, L0 + T, DL, seed=11)
    rc, rl = oracle(q_lat, q_rope, c, kr, L0, T)
    qc, rc_, cc, kc = q_lat.cuda(), q_rope.cuda(), c.cuda(), kr.cuda()
    outs = {}
    for ns in (1, 2, 5, 0, 49, 1000):
        ctx, lse = ops.prefill_cached(qc, rc_, cc, kc, L0, SCALE, False, ns)
        check_close(ctx.cpu().double(), rc, f"ctx ({ns} ranges)")
        torch.testing.assert_close(lse.cpu().double(), rl, rtol=0, atol=1e-3)
        outs[ns] = ctx
    # 1000 ranges are cut down to one per 32-key tile: the 49 tiles of L0 + T = 1540 keys
    assert torch.equal(outs[49], outs[1000])


def test_prefill_cached_rejects_bad_arguments(ops):
    q_lat, q_rope, c, kr = (t.cuda() for t in make(1, 4, 16, 10, 512, seed=6))
    with pytest.raises(ValueError):
        ops.prefill_cached(q_lat, q_rope, c, kr, 7, SCALE)  # L0 + T = 11 > 10 rows
    with pytest.raises(ValueError):
        ops.prefill_cached(q_lat, q_rope, c, kr.expand(1, 16, 10, 64), 2, SCALE)  # per-head k_rope
    with pytest.raises(ValueError):
        ops.prefill_cached(q_lat[..., :64], q_rope, c[..., :64], kr, 2, SCALE)  # d_latent 64 not built
    with pytest.raises(TypeError):
        ops.prefill_cached(q_lat.float(), q_rope, c, kr, 2, SCALE)
    with pytest.raises(RuntimeError):
        ops.prefill_cached(q_lat, q_rope, c, kr, 2, SCALE, False, -1)  # negative split count


def test_prefill_cached_is_deterministic(ops):
    q_lat, q_rope, c, kr = (t.cuda() for t in make(2, 20, 16, 700, 512, seed=8))
    a = ops.prefill_cached(q_lat, q_rope, c, kr, 680, SCALE)
    b = ops.prefill_cached(q_lat, q_rope, c, kr, 680, SCALE)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
