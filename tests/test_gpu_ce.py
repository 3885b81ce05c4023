"""GPU parity of the vocabulary-chunked linear cross-entropy (transformer.py:62-115):
the mla_ce_chunk kernel between hipBLASLt logit GEMMs, forward and backward, against the
oracle's restatement (fp64) and against the reference's own torch composition run on the
same bf16 logits."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import mla_oracle as O
from tests.gpu_util import randn_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ce():
    from transformer_amd import chunked_linear_cross_entropy
    return chunked_linear_cross_entropy


def reference_composition(x, w, y, chunk):
    """transformer.py:84-108 as written (bf16 logits, fp32 logsumexp / logaddexp), on the GPU."""
    xt, yt = x.reshape(-1, x.size(-1)), y.reshape(-1)
    lse = torch.full((xt.size(0),), float("-inf"), device=x.device)
    tl = torch.zeros(xt.size(0), device=x.device)
    for v0 in range(0, w.size(0), chunk):
        v1 = min(w.size(0), v0 + chunk)
        lf = (xt @ w[v0:v1].t()).float()
        lse = torch.logaddexp(lse, torch.logsumexp(lf, dim=-1))
        m = (yt >= v0) & (yt < v1)
        tl[m] = lf[m, yt[m] - v0]
    return lse - tl


@pytest.mark.parametrize("B,T,D,V,chunk", [(1, 1, 64, 8, 8), (2, 37, 64, 1000, 256), (3, 50, 128, 4096, 4096),
                                           (2, 64, 96, 2048, 1000)])
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_ce_forward_matches_oracle_and_reference(ce, B, T, D, V, chunk, reduction):
    print(f"case B={B} T={T} D={D} V={V} chunk={chunk} {reduction}", flush=True)
    g = torch.Generator().manual_seed(B * T + V)
    x = randn_bf16((B, T, D), g)
    w = randn_bf16((V, D), g, 3.0 / math.sqrt(D))
    y = torch.randint(0, V, (B, T), generator=g)
    got = ce(x.cuda(), w.cuda(), y.cuda(), chunk, reduction)
    per_row = ce(x.cuda(), w.cuda(), y.cuda(), chunk, "none").reshape(-1)
    ref_rows = reference_composition(x.cuda(), w.cuda(), y.cuda(), chunk)
    # the kernel on the same bf16 logits as the reference composition: fp32 agreement
    torch.testing.assert_close(per_row, ref_rows, rtol=1e-5, atol=1e-4)
    # against the fp64 oracle, whose logits are not rounded to bf16: rounding moves each logit by
    # at most 2^-9 of its size, so a row's loss (lse - target logit) by at most 2 * 2^-9 max|logit|
    orc = O.chunked_linear_cross_entropy(x.double(), w.double(), y, chunk, "none").reshape(-1)
    bound = 2.0 ** -8 * (x.double().reshape(-1, D) @ w.double().t()).abs().amax(-1) + 1e-4
    d = (per_row.cpu().double() - orc).abs()
    assert (d <= bound).all(), (d.max().item(), bound.min().item())
    red = {"mean": per_row.mean(), "sum": per_row.sum()}.get(reduction, per_row.view(B, T))
    torch.testing.assert_close(got, red, rtol=1e-6, atol=1e-5)


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_ce_backward_matches_fp64_autograd(ce, reduction):
    g = torch.Generator().manual_seed(77)
    B, T, D, V, chunk = 2, 29, 64, 520, 128
    x = randn_bf16((B, T, D), g)
    w = randn_bf16((V, D), g, 3.0 / math.sqrt(D))
    y = torch.randint(0, V, (B, T), generator=g)
    xg = x.cuda().requires_grad_(True)
    wg = w.cuda().requires_grad_(True)
    loss = ce(xg, wg, y.cuda(), chunk, reduction)
    up = torch.randn(loss.shape, generator=g) if reduction == "none" else torch.tensor(1.7)
    loss.backward(up.cuda().to(loss.dtype))
    xd = x.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    ref = O.chunked_linear_cross_entropy(xd, wd, y, chunk, reduction)
    ref.backward(up.double())
    for got, r, name in ((xg.grad, xd.grad, "dx"), (wg.grad, wd.grad, "dW")):
        scale = r.abs().max().item()
        err = (got.cpu().double() - r).abs()
        assert err.max() <= 2e-2 * scale and err.mean() <= 2e-3 * scale, (name, err.max().item(), scale)


def test_ce_training_shape_sampled(ce):
    # the benchmark dims (d_model 2048) and the reference's vocabulary (32768) in 4096-wide chunks
    g = torch.Generator(device="cuda").manual_seed(5)
    N, D, V = 2048, 2048, 32768
    x = torch.randn(1, N, D, generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn(V, D, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    y = torch.randint(0, V, (1, N), generator=g, device="cuda")
    rows = ce(x, w, y, 4096, "none").reshape(-1)
    ref = reference_composition(x, w, y, 4096)
    torch.testing.assert_close(rows, ref, rtol=1e-5, atol=1e-4)
    full = F.cross_entropy((x.reshape(N, D) @ w.t()).float(), y.reshape(N), reduction="none")
    torch.testing.assert_close(rows, full, rtol=1e-5, atol=1e-4)


def test_ce_under_torch_compile_matches_eager(ce):
    # the reference compiles its model with fullgraph=False (train.py:222-227)
    g = torch.Generator().manual_seed(8)
    x = randn_bf16((2, 33, 64), g).cuda().requires_grad_(True)
    w = randn_bf16((512, 64), g, 0.3).cuda().requires_grad_(True)
    y = torch.randint(0, 512, (2, 33), generator=g).cuda()
    fn = torch.compile(lambda a, b: ce(a, b, y, 128, "mean"), fullgraph=False)
    loss_c = fn(x, w)
    loss_c.backward()
    gx, gw = x.grad.clone(), w.grad.clone()
    x.grad = w.grad = None
    loss_e = ce(x, w, y, 128, "mean")
    loss_e.backward()
    torch.testing.assert_close(loss_c, loss_e, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(gx, x.grad, rtol=0, atol=0)
    torch.testing.assert_close(gw, w.grad, rtol=0, atol=0)


def test_ce_fp32_outside_autocast_matches_oracle(ce):
    # an fp32 caller outside autocast: the reference computes the logits, the loss and the
    # gradients in fp32 (transformer.py:96-98); so does the kernel path (fp32 logits)
    g = torch.Generator().manual_seed(61)
    B, T, D, V, chunk = 2, 40, 128, 3000, 512
    x = torch.randn(B, T, D, generator=g)
    w = torch.randn(V, D, generator=g) * (3.0 / math.sqrt(D))
    y = torch.randint(0, V, (B, T), generator=g)
    xg, wg = x.cuda().requires_grad_(True), w.cuda().requires_grad_(True)
    loss = ce(xg, wg, y.cuda(), chunk, "mean")
    assert loss.dtype == torch.float32
    loss.backward()
    xo, wo = x.double().requires_grad_(True), w.double().requires_grad_(True)
    lo = O.chunked_linear_cross_entropy(xo, wo, y, chunk, "mean")
    lo.backward()
    torch.testing.assert_close(loss.detach().cpu().double(), lo.detach(), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(xg.grad.cpu().double(), xo.grad, rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(wg.grad.cpu().double(), wo.grad, rtol=1e-4, atol=1e-6)


def test_ce_input_gradient_accumulates_in_fp32_under_autocast(ce):
    # 16 chunks: the input gradient is summed over the chunks in fp32, as autograd sums the
    # reference's per-chunk bf16 products (transformer.py:84-108 under autocast); summing in
    # bf16 instead rounds 16 times and misses this bound
    g = torch.Generator().manual_seed(62)
    B, T, D, V, chunk = 2, 64, 128, 4096, 256
    x = torch.randn(B, T, D, generator=g)
    w = torch.randn(V, D, generator=g) * (3.0 / math.sqrt(D))
    y = torch.randint(0, V, (B, T), generator=g)
    grads = []
    for fn in ("ours", "reference"):
        xg, wg = x.cuda().requires_grad_(True), w.cuda().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            if fn == "ours":
                loss = ce(xg, wg, y.cuda(), chunk, "mean")
            else:
                loss = reference_composition(xg, wg, y.cuda(), chunk).mean()
        loss.backward()
        assert xg.grad.dtype == torch.float32
        grads.append(xg.grad.cpu().double())
    scale = grads[1].abs().max().item()
    err = (grads[0] - grads[1]).abs().max().item()
    assert err <= 2e-3 * scale, (err, scale)
