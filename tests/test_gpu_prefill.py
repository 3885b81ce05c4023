"""GPU parity of the causal prefill forward (mla_prefill_fwd) against the oracle's
attention (restating SDPA at transformer.py:311-314 and the masked absorbed
prefill at :273-291).

Tolerance: bf16 output within max-abs 2e-2 and mean-abs 2e-3 of the
fp64 oracle on the same bf16 inputs; softmax row sums, recomputed from the
kernel's LSE in fp64, within 1e-3 of 1.
"""
import math

import pytest
import torch

from oracle import mla_oracle as O
from tests.gpu_util import MAX_ABS, MEAN_ABS, ROWSUM_TOL, check_close, randn_bf16, rowsum_from_lse

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import transformer_amd  # noqa: F401
    return torch.ops.mla_mi355x


def make_inputs(B, Tq, Tk, H, Hr, dn, seed, q_scale=1.0, dv=128):
    g = torch.Generator().manual_seed(seed)
    return dict(
        q_nope=randn_bf16((B, Tq, H, dn), g, q_scale), q_rope=randn_bf16((B, Tq, H, 64), g, q_scale),
        k_nope=randn_bf16((B, Tk, H, dn), g), k_rope=randn_bf16((B, Tk, Hr, 64), g),
        v=randn_bf16((B, Tk, H, dv), g))


def oracle(inp, scale, causal, q_offset, heads=None):
    """fp64 oracle O [B,Tq,H,dv], LSE [B,H,Tq] (optionally a subset of (b, h) pairs)."""
    q = torch.cat([inp["q_nope"], inp["q_rope"]], -1).double().transpose(1, 2)  # [B,H,Tq,D]
    kr = inp["k_rope"].double().transpose(1, 2)
    H = q.shape[1]
    k = torch.cat([inp["k_nope"].double().transpose(1, 2), kr.expand(-1, H, -1, -1)], -1)
    v = inp["v"].double().transpose(1, 2)
    if heads is not None:
        outs = {}
        for b, h in heads:
            o, lse = O.attention(q[b, h], k[b, h], v[b, h], scale, causal, q_offset)
            outs[(b, h)] = (o, lse)
        return outs
    o, lse = O.attention(q, k, v, scale, causal, q_offset)
    return o.transpose(1, 2), lse


def run(ops, inp, scale, causal=True, q_offset=0):
    d = {k: v.cuda() for k, v in inp.items()}
    o, lse = ops.prefill_fwd(d["q_nope"], d["q_rope"], d["k_nope"], d["k_rope"], d["v"], scale, causal, q_offset)
    torch.cuda.synchronize()
    return o.cpu(), lse.cpu()


CASES = [
    # B, Tq, Tk, H, Hr, dn, causal, q_offset
    (1, 1, 1, 1, 1, 128, True, 0),
    (2, 7, 7, 3, 1, 128, True, 0),
    (1, 64, 64, 2, 2, 128, True, 0),
    (2, 130, 130, 2, 1, 128, True, 0),
    (1, 257, 257, 3, 3, 64, True, 0),
    (1, 200, 200, 2, 1, 64, False, 0),
    (2, 5, 83, 2, 1, 128, True, 78),   # chunked prefill: bottom-right mask
    (1, 1, 300, 4, 4, 64, True, 299),  # single query against a long cache
    (1, 129, 40, 2, 1, 128, False, 0),  # Tk < Tq, no mask
]


@pytest.mark.parametrize("B,Tq,Tk,H,Hr,dn,causal,q_offset", CASES)
def test_prefill_fwd_matches_oracle(ops, B, Tq, Tk, H, Hr, dn, causal, q_offset):
    print(f"case B={B} Tq={Tq} Tk={Tk} H={H} Hr={Hr} dn={dn} causal={causal} q_offset={q_offset}", flush=True)
    inp = make_inputs(B, Tq, Tk, H, Hr, dn, seed=Tq * 31 + Tk)
    scale = 1 / math.sqrt(dn + 64)
    o, lse = run(ops, inp, scale, causal, q_offset)
    ref_o, ref_lse = oracle(inp, scale, causal, q_offset)
    check_close(o.double(), ref_o, "O")
    torch.testing.assert_close(lse.double(), ref_lse, rtol=0, atol=1e-3)


def test_prefill_fwd_peaked_and_rowsums(ops):
    # Q scaled x8: attention concentrates, so the tolerance is not met by near-uniform rows
    inp = make_inputs(1, 256, 256, 2, 1, 128, seed=5, q_scale=8.0)
    scale = 1 / math.sqrt(192)
    o, lse = run(ops, inp, scale)
    ref_o, _ = oracle(inp, scale, True, 0)
    check_close(o.double(), ref_o, "O (peaked)")
    q = torch.cat([inp["q_nope"], inp["q_rope"]], -1)[0, :, 0]
    k = torch.cat([inp["k_nope"][0, :, 0], inp["k_rope"][0, :, 0]], -1)
    sums = rowsum_from_lse(q, k, lse[0, 0], scale, True, 0, rows=[0, 1, 63, 64, 127, 200, 255])
    assert max(abs(s - 1) for s in sums) <= ROWSUM_TOL, sums


def test_prefill_fwd_v_ones_gives_ones(ops):
    inp = make_inputs(2, 150, 150, 2, 1, 128, seed=6)
    inp["v"] = torch.ones_like(inp["v"])
    o, _ = run(ops, inp, 1 / math.sqrt(192))
    assert (o.float() - 1).abs().max().item() <= 1e-2


def test_prefill_fwd_strided_views_like_the_module(ops):
    # q_rope / k_rope as views into one [B, T, H + 1, 64] rope buffer, q_nope / k_nope / v as
    # views of projection outputs: no copies are made on the way into the kernel
    g = torch.Generator().manual_seed(12)
    B, T, H = 2, 96, 4
    roped = randn_bf16((B, T, H + 1, 64), g).cuda()
    kv = randn_bf16((B, T, H * 256), g).cuda()
    qn = randn_bf16((B, T, H * 128), g).cuda().view(B, T, H, 128)
    kn = kv.view(B, T, H, 256)[..., :128]
    v = kv.view(B, T, H, 256)[..., 128:]
    scale = 1 / math.sqrt(192)
    o, lse = ops.prefill_fwd(qn, roped[:, :, :H], kn, roped[:, :, H:], v, scale, True, 0)
    inp = dict(q_nope=qn.cpu(), q_rope=roped[:, :, :H].cpu(), k_nope=kn.cpu(), k_rope=roped[:, :, H:].cpu(),
               v=v.cpu())
    ref_o, _ = oracle(inp, scale, True, 0)
    check_close(o.cpu().double(), ref_o, "O (strided)")


def test_prefill_fwd_is_deterministic(ops):
    inp = {k: v.cuda() for k, v in make_inputs(1, 300, 300, 2, 1, 128, seed=13).items()}
    a = ops.prefill_fwd(inp["q_nope"], inp["q_rope"], inp["k_nope"], inp["k_rope"], inp["v"], 0.1, True, 0)
    b = ops.prefill_fwd(inp["q_nope"], inp["q_rope"], inp["k_nope"], inp["k_rope"], inp["v"], 0.1, True, 0)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_prefill_fwd_config1_shape_sampled_heads(ops):
    # the benchmark prefill shape (B=12, T=2048, H=16, d_qk=192, d_v=128, shared k_rope): the full
    # launch runs, and sampled (b, h) pairs are checked against the oracle.
    B, T, H = 12, 2048, 16
    inp = make_inputs(B, T, T, H, 1, 128, seed=2024)
    scale = 1 / math.sqrt(192)
    o, lse = run(ops, inp, scale)
    pairs = [(0, 0), (5, 7), (11, 15)]
    ref = oracle(inp, scale, True, 0, heads=pairs)
    for (b, h), (ro, rl) in ref.items():
        check_close(o[b, :, h].double(), ro, f"O[b={b},h={h}]")
        torch.testing.assert_close(lse[b, h].double(), rl, rtol=0, atol=1e-3)


def test_prefill_fwd_late_score_jump_takes_the_rescaling_path(ops):
    # Scores of key 100 exceed every score of the first 64 keys by ~200 in log2 units, so
    # the kernel's fixed first-tile reference max would overflow; the workgroup must
    # notice and recompute with the rescaling loop.  Checked against the fp64 oracle.
    inp = make_inputs(1, 160, 160, 2, 1, 128, seed=17)
    q = torch.cat([inp["q_nope"], inp["q_rope"]], -1).float()  # [1, T, H, 192]
    k_jump = (8.0 * q[0, 120, 0]).to(torch.bfloat16)            # aligned with query 120 of head 0
    inp["k_nope"][0, 100, 0] = k_jump[:128]
    inp["k_rope"][0, 100, 0] = k_jump[128:]
    scale = 1 / math.sqrt(192)
    o, lse = run(ops, inp, scale)
    ref_o, ref_lse = oracle(inp, scale, True, 0)
    assert torch.isfinite(o.float()).all() and torch.isfinite(lse).all()
    check_close(o.double(), ref_o, "O (score jump)")
    torch.testing.assert_close(lse.double(), ref_lse, rtol=0, atol=1e-3)
    # and the jump really is beyond the fast path's range for some row
    qk = (q[0, 100:, 0] @ k_jump.float()) * scale * 1.4426950408889634
    assert qk.max().item() > 130


def test_prefill_fwd_rescaling_path_in_a_q_tile_that_preloads_the_next(ops):
    # T = 256: one workgroup runs q-tile 1 (rows 128..255, 8 key tiles, whose last steps load
    # q-tile 0's first key tiles) and then q-tile 0.  The score jump sits in q-tile 1, so its
    # recomputation must reload its own tiles and leave q-tile 0 correct.
    inp = make_inputs(1, 256, 256, 2, 1, 128, seed=19)
    q = torch.cat([inp["q_nope"], inp["q_rope"]], -1).float()
    k_jump = (8.0 * q[0, 200, 1]).to(torch.bfloat16)  # aligned with query 200 of head 1
    inp["k_nope"][0, 150, 1] = k_jump[:128]
    inp["k_rope"][0, 150, 0] = k_jump[128:]  # shared k_rope row: every head sees it
    scale = 1 / math.sqrt(192)
    o, lse = run(ops, inp, scale)
    ref_o, ref_lse = oracle(inp, scale, True, 0)
    assert torch.isfinite(o.float()).all() and torch.isfinite(lse).all()
    check_close(o.double(), ref_o, "O (score jump, preloading q-tile)")
    torch.testing.assert_close(lse.double(), ref_lse, rtol=0, atol=1e-3)
    qk = (q[0, 150:, 1] @ torch.cat([k_jump[:128], k_jump[128:]]).float()) * scale * 1.4426950408889634
    assert qk.max().item() > 130


def test_prefill_fwd_rejects_bad_shapes(ops):
    inp = {k: v.cuda() for k, v in make_inputs(1, 8, 8, 2, 1, 128, seed=1).items()}
    with pytest.raises(ValueError):
        ops.prefill_fwd(inp["q_nope"], inp["q_rope"], inp["k_nope"][:, :4], inp["k_rope"], inp["v"], 0.1, True, 0)
    with pytest.raises(TypeError):
        ops.prefill_fwd(inp["q_nope"].float(), inp["q_rope"], inp["k_nope"], inp["k_rope"], inp["v"], 0.1, True, 0)
