"""Seeded random-shape sweeps of the HIP entry points against the oracle.

Shapes are drawn from a fixed generator (the same on every run) over the ranges the
kernels branch on: ragged lengths around the 32-row blocks and 128-row tiles, q_offset
(chunked prefill and decode-like single queries), causal and full masks, shared and
per-head k_rope, nope 64 / 128, head counts that leave a partial head group, latent
widths 64..512, split counts, and per-sequence lengths including 0; RMSNorm rows of any
multiple-of-8 width up to 4096 (partial lane chunks, bf16 and fp32 rows, eps 0 and up), and
the chunked cross-entropy with vocabulary and chunk widths that do and do not divide each
other.  Each case prints its shape before running, so a failure names it.

Tolerances are the path's bf16 bound (max-abs 2e-2, mean-abs 2e-3 against the fp64 oracle on
the same bf16 inputs; gradients relative to their scale).
"""
import math
import random

import pytest
import torch

from tests.gpu_util import check_close, randn_bf16
from tests.test_gpu_backward import check_grad, oracle_grads, run_bwd
from tests.test_gpu_decode import make as make_decode
from tests.test_gpu_decode import oracle as decode_oracle
from tests.test_gpu_decode import run as run_decode
from tests.test_gpu_prefill import make_inputs, oracle, run

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import transformer_amd  # noqa: F401
    return torch.ops.mla_mi355x


def _prefill_cases(n, seed):
    rng = random.Random(seed)
    cases = []
    for _ in range(n):
        causal = rng.random() < 0.75
        Tq = rng.choice([1, 2, 31, 32, 33, 95, 127, 128, 129, 200, 255, 256, 257])
        if causal and rng.random() < 0.4:
            q_offset = rng.choice([1, 17, 64, 100])
            Tk = Tq + q_offset
        else:
            q_offset = 0
            Tk = Tq if causal else rng.choice([1, 33, 64, 150, 260])
        H = rng.choice([1, 2, 3])
        Hr = rng.choice([1, H])
        dn = rng.choice([64, 128])
        B = rng.choice([1, 2])
        cases.append((B, Tq, Tk, H, Hr, dn, causal, q_offset))
    return cases


PREFILL = _prefill_cases(14, seed=2024)


@pytest.mark.parametrize("B,Tq,Tk,H,Hr,dn,causal,q_offset", PREFILL)
def test_prefill_forward_sweep(ops, B, Tq, Tk, H, Hr, dn, causal, q_offset):
    print(f"case B={B} Tq={Tq} Tk={Tk} H={H} Hr={Hr} dn={dn} causal={causal} q_offset={q_offset}", flush=True)
    inp = make_inputs(B, Tq, Tk, H, Hr, dn, seed=B * 1000 + Tq * 7 + Tk)
    scale = 1 / math.sqrt(dn + 64)
    o, lse = run(ops, inp, scale, causal, q_offset)
    ro, rl = oracle(inp, scale, causal, q_offset)
    check_close(o.double(), ro, "O")
    torch.testing.assert_close(lse.double(), rl, rtol=0, atol=1e-3)


@pytest.mark.parametrize("B,Tq,Tk,H,Hr,dn,causal,q_offset", PREFILL[:10])
def test_prefill_backward_sweep_both_dq_paths(ops, monkeypatch, B, Tq, Tk, H, Hr, dn, causal, q_offset):
    print(f"case B={B} Tq={Tq} Tk={Tk} H={H} Hr={Hr} dn={dn} causal={causal} q_offset={q_offset}", flush=True)
    from transformer_amd import kernels
    inp = make_inputs(B, Tq, Tk, H, Hr, dn, seed=B * 1000 + Tq * 5 + Tk)
    do = randn_bf16((B, Tq, H, 128), torch.Generator().manual_seed(Tq + Tk))
    scale = 1 / math.sqrt(dn + 64)
    ref = oracle_grads(inp, do, scale, causal, q_offset)
    for stored in (True, False):
        monkeypatch.setattr(kernels, "BWD_STORED_DS", stored)
        got = run_bwd(ops, inp, do, scale, causal, q_offset)
        for name in ref:
            assert got[name].shape == ref[name].shape, name
            check_grad(got[name], ref[name], f"{name} (stored dS: {stored})")


def _decode_cases(n, seed):
    rng = random.Random(seed)
    cases = []
    for _ in range(n):
        B = rng.choice([1, 2, 3, 5])
        H = rng.choice([1, 5, 16, 17, 32])
        L = rng.choice([1, 15, 64, 65, 300, 777, 1500])
        DL = rng.choice([64, 128, 256, 384, 512])
        Hr = rng.choice([1, H])
        splits = rng.choice([0, 0, 1, 3, 8])
        lens = None
        if rng.random() < 0.5:
            lens = [rng.choice([0, 1, L // 3, L - 1, L]) for _ in range(B)]
            lens = [max(0, x) for x in lens]
        cases.append((B, H, L, DL, Hr, splits, lens))
    return cases


@pytest.mark.parametrize("B,H,L,DL,Hr,splits,lens", _decode_cases(14, seed=7))
def test_decode_sweep(ops, B, H, L, DL, Hr, splits, lens):
    print(f"case B={B} H={H} L={L} DL={DL} Hr={Hr} splits={splits} lens={lens}", flush=True)
    q_lat, q_rope, c, kr = make_decode(B, H, L, DL, Hr, seed=B * 31 + H * 7 + L + DL)
    scale = 1 / math.sqrt(192)
    ctx, lse = run_decode(ops, q_lat, q_rope, c, kr, scale, seq_lens=lens, splits=splits)
    for b in range(B):
        n = L if lens is None else lens[b]
        if n == 0:  # an empty sequence: zero context, LSE -inf
            assert (ctx[b] == 0).all() and torch.isinf(lse[b]).all() and (lse[b] < 0).all()
            continue
        rc, rl = decode_oracle(q_lat[b:b + 1], q_rope[b:b + 1], c[b:b + 1, :n], kr[b:b + 1, :, :n], scale)
        check_close(ctx[b:b + 1].double(), rc, f"ctx (b={b}, len={n})")
        torch.testing.assert_close(lse[b:b + 1].double(), rl, rtol=0, atol=1e-3)


# ---------------------------------------------------------------- RMSNorm and the cross-entropy chunk kernel

def _rms_cases(n, seed):
    rng = random.Random(seed)
    return [(rng.choice([1, 3, 4, 5, 63, 64, 65, 257, 1031]), 8 * rng.randint(1, 512),
             rng.choice([torch.bfloat16, torch.float32]), rng.choice([0.0, 1e-6, 1e-2])) for _ in range(n)]


@pytest.mark.parametrize("M,K,dtype,eps", _rms_cases(10, 1234))
def test_sweep_rmsnorm_forward_backward(ops, M, K, dtype, eps):
    from oracle import mla_oracle as O
    print(f"case rmsnorm M={M} K={K} {dtype} eps={eps}", flush=True)
    g = torch.Generator().manual_seed(M * 8191 + K)
    x = (torch.randn(M, K, generator=g) * 2).to(dtype)
    w = torch.randn(K, generator=g)
    dy = randn_bf16((M, K), g)
    y, r = ops.rmsnorm(x.cuda(), w.cuda(), eps)
    ref = O.rms_norm(x.double(), w.double(), eps)
    assert ((y.cpu().double() - ref).abs() <= ref.abs() * 2.0 ** -7 + 1e-30).all(), "beyond one bf16 ulp"
    dx, dw = ops.rmsnorm_bwd(dy.cuda(), x.cuda(), w.cuda(), r)
    dx_ref, dw_ref = O.rms_norm_bwd(x.double(), w.double(), dy.double(), eps)
    sx = max(1.0, dx_ref.abs().max().item())
    check_close(dx.float(), dx_ref, "dx", max_abs=2e-2 * sx, mean_abs=2e-3 * sx)
    torch.testing.assert_close(dw.cpu().double(), dw_ref, rtol=1e-4, atol=1e-5 * dw_ref.abs().max().item())


def _ce_cases(n, seed):
    rng = random.Random(seed)
    cases = []
    for _ in range(n):
        V = 8 * rng.randint(1, 600)
        cases.append((rng.choice([1, 2, 7, 64, 129, 300]), V, 8 * rng.randint(1, 600), rng.choice([0.5, 3.0, 12.0])))
    return cases


@pytest.mark.parametrize("N,V,chunk,spread", _ce_cases(10, 4321))
def test_sweep_ce_chunks_match_full_softmax(N, V, chunk, spread):
    # the chunked loss and its gradient against F.cross_entropy on the full bf16 logits
    import torch.nn.functional as F
    from transformer_amd import chunked_linear_cross_entropy
    print(f"case ce N={N} V={V} chunk={chunk} spread={spread}", flush=True)
    g = torch.Generator().manual_seed(N * 131 + V)
    D = 64
    x = randn_bf16((1, N, D), g).cuda().requires_grad_(True)
    w = randn_bf16((V, D), g, spread / math.sqrt(D)).cuda()
    y = torch.randint(0, V, (1, N), generator=g).cuda()
    rows = chunked_linear_cross_entropy(x, w, y, chunk, "none").reshape(-1)
    logits = (x.detach().reshape(N, D) @ w.t()).float()
    ref = F.cross_entropy(logits, y.reshape(N), reduction="none")
    torch.testing.assert_close(rows, ref, rtol=1e-5, atol=1e-4)
    rows.sum().backward()
    p = torch.softmax(logits, -1)
    p[torch.arange(N), y.reshape(N)] -= 1.0
    dx_ref = (p @ w.float()).reshape(1, N, D)
    scale = dx_ref.abs().max().item()
    err = (x.grad.float() - dx_ref).abs()
    assert err.max() <= 2e-2 * scale and err.mean() <= 2e-3 * scale, (err.max().item(), scale)
