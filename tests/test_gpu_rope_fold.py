"""GPU tests of the RoPE fold: prefill_fwd_rope rotates the queries' rope slice in the attention
kernel's Q load (transformer.py:228-233 folded into :314) and its backward rotates dq_rope back in
the dQ kernel's epilogue.

Against the unfused composition (the RoPE kernel over the q heads, then prefill_fwd, autograd
through both), on the same bf16 inputs: O, LSE and the rotated slice are bit for bit equal (the
rotation is the same fp32 arithmetic with one rounding); dq_nope, dk and dv are bit for bit equal;
dq_rope differs by a few bf16 roundings (the fold rotates the fp32 gradient before rounding, the
composition rounds, rotates, rounds again), checked within 3 roundings of each rotation pair's
magnitude and against the fp64 oracle of the whole chain at the path's bound.  At the module level, the bf16
training step with the fold on and off gives bitwise equal outputs and gradients within the bound.
"""
import math

import pytest
import torch

from oracle import mla_oracle as O
from tests.gpu_util import check_close, randn_bf16
from tests.test_gpu_backward import check_grad

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import transformer_amd  # noqa: F401
    return torch.ops.mla_mi355x


def _inputs(B, T, H, seed):
    g = torch.Generator().manual_seed(seed)
    return dict(q_nope=randn_bf16((B, T, H, 128), g), q_raw=randn_bf16((B, T, H, 64), g),
                k_nope=randn_bf16((B, T, H, 128), g), k_rope=randn_bf16((B, T, 1, 64), g),
                v=randn_bf16((B, T, H, 128), g), do=randn_bf16((B, T, H, 128), g))


CASES = [
    # B, T, H, pos_offset
    (2, 300, 3, 0),
    (1, 1024, 2, 0),     # a small grid: the key split (the first segment of a q-tile stores the rotated rows)
    (3, 260, 4, 517),    # positions from 517 on (a cache passed with use_cache=False keeps q_offset 0)
]


@pytest.mark.parametrize("B,T,H,pos", CASES)
def test_fold_equals_the_unfused_composition(ops, B, T, H, pos):
    print(f"case B={B} T={T} H={H} pos_offset={pos}", flush=True)
    x = {k: v.cuda() for k, v in _inputs(B, T, H, seed=T + pos).items()}
    cos, sin = O.rope_tables(64, 4096)
    cos, sin = cos.to(torch.bfloat16).cuda(), sin.to(torch.bfloat16).cuda()
    scale = 1 / math.sqrt(192)
    leaves = {k: x[k].clone().requires_grad_(True) for k in ("q_nope", "q_raw", "k_nope", "k_rope", "v")}
    o_f, lse_f, q_rot = ops.prefill_fwd_rope(leaves["q_nope"], leaves["q_raw"], leaves["k_nope"], leaves["k_rope"],
                                             leaves["v"], cos, sin, scale, True, 0, pos, True)
    o_f.backward(x["do"])
    leaves_u = {k: x[k].clone().requires_grad_(True) for k in ("q_nope", "q_raw", "k_nope", "k_rope", "v")}
    q_rope_u = ops.rope(leaves_u["q_raw"], cos, sin, pos, False)
    o_u, lse_u = ops.prefill_fwd(leaves_u["q_nope"], q_rope_u, leaves_u["k_nope"], leaves_u["k_rope"], leaves_u["v"],
                                 scale, True, 0)
    o_u.backward(x["do"])
    torch.cuda.synchronize()
    assert torch.equal(q_rot, q_rope_u.detach()), "rotated slice differs from the RoPE kernel's"
    assert torch.equal(o_f, o_u) and torch.equal(lse_f, lse_u), "forward differs from the composition"
    for k in ("q_nope", "k_nope", "k_rope", "v"):
        assert torch.equal(leaves[k].grad, leaves_u[k].grad), f"d{k} differs from the composition"
    # the composition rounds the rotated gradient (dy1, dy2) to bf16 before rotating it back, so the
    # two differ by a few bf16 roundings of the pair's magnitude |(dy1, dy2)| = |(g_i, g_{i+32})|
    gf, gu = leaves["q_raw"].grad.float(), leaves_u["q_raw"].grad.float()
    mag = torch.sqrt(gu[..., :32] ** 2 + gu[..., 32:] ** 2).repeat(1, 1, 1, 2)
    bound = 3 * mag * 2.0 ** -8 + 1e-30
    assert ((gf - gu).abs() <= bound).all(), \
        f"dq_rope beyond 3 bf16 roundings of the pair magnitude: {((gf - gu).abs() / bound).max().item():.3f} x"
    # the whole chain against fp64 autograd of the oracle (rotation, attention)
    c64, s64 = O.rope_tables(64, 4096)
    q_raw = x["q_raw"].double().cpu().requires_grad_(True)
    qr = O.apply_rope(q_raw.transpose(1, 2), c64[pos:pos + T].double(), s64[pos:pos + T].double())  # [B,H,T,64]
    q = torch.cat([x["q_nope"].double().cpu().transpose(1, 2), qr], -1)
    k = torch.cat([x["k_nope"].double().cpu().transpose(1, 2),
                   x["k_rope"].double().cpu().transpose(1, 2).expand(-1, H, -1, -1)], -1)
    o_ref, _ = O.attention(q, k, x["v"].double().cpu().transpose(1, 2), scale, True, 0)
    o_ref.backward(x["do"].double().cpu().transpose(1, 2))
    check_close(o_f.detach().cpu().double(), o_ref.detach().transpose(1, 2), "O (fold)")
    check_grad(leaves["q_raw"].grad.cpu(), q_raw.grad, "dq_rope (fold, unrotated slice)")


def test_fold_without_saving_the_rotated_slice(ops):
    x = {k: v.cuda() for k, v in _inputs(1, 200, 2, seed=5).items()}
    cos, sin = O.rope_tables(64, 1024)
    cos, sin = cos.to(torch.bfloat16).cuda(), sin.to(torch.bfloat16).cuda()
    with torch.no_grad():
        o, lse, q_rot = ops.prefill_fwd_rope(x["q_nope"], x["q_raw"], x["k_nope"], x["k_rope"], x["v"], cos, sin,
                                             0.07, True, 0, 3, False)
        o_u, lse_u = ops.prefill_fwd(x["q_nope"], ops.rope(x["q_raw"], cos, sin, 3, False), x["k_nope"],
                                     x["k_rope"], x["v"], 0.07, True, 0)
    assert q_rot.numel() == 0 and torch.equal(o, o_u) and torch.equal(lse, lse_u)
    with pytest.raises(ValueError):  # positions past the table
        ops.prefill_fwd_rope(x["q_nope"], x["q_raw"], x["k_nope"], x["k_rope"], x["v"], cos, sin, 0.07, True, 0,
                             900, False)


def test_module_training_step_with_and_without_the_fold():
    # the module's bf16 training step (autocast, transformer.py:306-316 with norm1 in front, as in
    # TransformerBlock): outputs bitwise equal with the fold on and off, gradients within the bound
    import transformer_amd.mla as M
    from tests.test_gpu_module import _baseline_module
    m, args = _baseline_module(seed=61)
    g = torch.Generator().manual_seed(62)
    x = torch.randn(2, 512, args.d_model, generator=g).cuda()
    dy = torch.randn(2, 512, args.d_model, generator=g).cuda()

    def step(fold):
        saved = M.ROPE_FOLD
        M.ROPE_FOLD = fold
        try:
            m.zero_grad(set_to_none=True)
            xi = x.clone().requires_grad_(True)
            with torch.autocast("cuda", dtype=torch.bfloat16):
                y, _ = m(xi)
            y.float().backward(dy)
            torch.cuda.synchronize()
            return y.detach(), xi.grad.detach(), {n: p.grad.detach().clone() for n, p in m.named_parameters()}
        finally:
            M.ROPE_FOLD = saved

    y1, gx1, gp1 = step(True)
    y0, gx0, gp0 = step(False)
    assert torch.equal(y1, y0), "module output differs with the fold"
    check_grad(gx1.cpu().double(), gx0.cpu().double(), "d x (fold vs unfused)")
    # weight gradients sum B T = 1024 tokens' products, so the per-element bf16 roundings by which
    # the two dq_rope differ add up: the absolute bound is doubled for them (their rms is ~1); the
    # relative bounds of check_grad hold as for every gradient
    for n in gp0:
        check_grad(gp1[n].cpu().double(), gp0[n].cpu().double(), f"d {n} (fold vs unfused)", factor=2.0)
