"""GPU parity of the RMSNorm kernels (mla_rmsnorm, mla_rmsnorm_bwd) in front of the MLA
down-projections, against the oracle's rms_norm / rms_norm_bwd (transformer.py:16-27) and
the reference's fused RMSNorm + down-projection self-test (fused_mla_triton_kernels.py:
800-829: seed 42, M=512, K=1792, N=384, mean < 1e-3, p99 < 0.1, max < 0.5)."""
import pytest
import torch

from oracle import mla_oracle as O
from tests.gpu_util import check_close, randn_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import transformer_amd  # noqa: F401
    return torch.ops.mla_mi355x


def _bf16_ulp_close(got, ref, what, frac_limit=1e-3):
    """got (bf16) within one bf16 ulp of the fp64 reference everywhere, and equal to its
    rounding except for a small fraction (rounding ties moved by fp32 sum order)."""
    ref_b = ref.to(torch.bfloat16).double()
    g = got.double()
    ulp = ref.abs().clamp_min(1e-30) * 2.0 ** -7
    assert ((g - ref).abs() <= ulp).all(), f"{what}: beyond one bf16 ulp: max {(g - ref).abs().max():.3e}"
    frac = (g != ref_b).double().mean().item()
    assert frac <= frac_limit, f"{what}: {frac:.2e} of the elements differ from the rounded reference"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,K", [(1, 8), (7, 1792), (33, 2048), (130, 4096), (5, 520), (2049, 512)])
def test_rmsnorm_forward_matches_oracle(ops, dtype, M, K):
    g = torch.Generator().manual_seed(M * 7 + K)
    x = (torch.randn(M, K, generator=g) * 3).to(dtype)
    w = torch.randn(K, generator=g)
    y, r = ops.rmsnorm(x.cuda(), w.cuda(), 1e-6)
    ref = O.rms_norm(x.double(), w.double(), 1e-6)
    _bf16_ulp_close(y.cpu(), ref, f"y {dtype} M={M} K={K}")
    r_ref = x.double().pow(2).mean(-1).add(1e-6).rsqrt()
    torch.testing.assert_close(r.cpu().double(), r_ref, rtol=2e-6, atol=0)


def test_rmsnorm_strided_rows_batched_shape_and_empty(ops):
    g = torch.Generator().manual_seed(5)
    buf = randn_bf16((3, 11, 2048 + 64), g).cuda()
    x = buf[..., 32:32 + 2048]  # rows of stride 2112, 64-byte offset
    w = torch.rand(2048, generator=g).cuda()
    y, r = ops.rmsnorm(x, w, 1e-5)
    assert y.shape == (3, 11, 2048) and r.shape == (3, 11)
    _bf16_ulp_close(y.cpu(), O.rms_norm(x.cpu().double(), w.cpu().double(), 1e-5), "strided")
    y0, r0 = ops.rmsnorm(x[:0], w, 1e-5)
    assert y0.shape == (0, 11, 2048) and r0.shape == (0, 11)
    with pytest.raises(ValueError):
        ops.rmsnorm(torch.zeros(4, 12, device="cuda"), torch.ones(12, device="cuda"), 1e-6)  # K % 8


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,K", [(3, 64), (37, 1792), (1000, 2048), (4100, 512)])
def test_rmsnorm_backward_matches_oracle(ops, dtype, M, K):
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g).to(dtype)
    w = torch.randn(K, generator=g)
    dy = randn_bf16((M, K), g)
    _, r = ops.rmsnorm(x.cuda(), w.cuda(), 1e-6)
    dx, dw = ops.rmsnorm_bwd(dy.cuda(), x.cuda(), w.cuda(), r)
    dx_ref, dw_ref = O.rms_norm_bwd(x.double(), w.double(), dy.double(), 1e-6)
    assert dx.dtype == dtype and dw.dtype == torch.float32
    if dtype == torch.float32:
        torch.testing.assert_close(dx.cpu().double(), dx_ref, rtol=1e-4, atol=1e-5)
    else:
        check_close(dx.float(), dx_ref, f"dx M={M} K={K}", max_abs=2e-2 * max(1.0, dx_ref.abs().max().item()))
    scale = dw_ref.abs().max().item()
    torch.testing.assert_close(dw.cpu().double(), dw_ref, rtol=1e-4, atol=1e-5 * scale)
    dx2, dw2 = ops.rmsnorm_bwd(dy.cuda(), x.cuda(), w.cuda(), r)
    assert torch.equal(dx, dx2) and torch.equal(dw, dw2), "backward is not bitwise reproducible"


def test_rmsnorm_module_autograd_under_autocast():
    from transformer_amd import RMSNorm
    g = torch.Generator().manual_seed(9)
    norm = RMSNorm(1792).cuda()
    with torch.no_grad():
        norm.weight.copy_(torch.randn(1792, generator=g))
    x = torch.randn(2, 50, 1792, generator=g).cuda().requires_grad_(True)  # fp32 residual stream
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = norm(x)
    assert y.dtype == torch.bfloat16
    dy = randn_bf16((2, 50, 1792), g)
    y.backward(dy.cuda())
    ref = O.rms_norm(x.detach().cpu().double(), norm.weight.detach().cpu().double(), 1e-6)
    _bf16_ulp_close(y.detach().cpu(), ref, "module y")
    dx_ref, dw_ref = O.rms_norm_bwd(x.detach().cpu(), norm.weight.detach().cpu(), dy.double(), 1e-6)
    torch.testing.assert_close(x.grad.cpu().double(), dx_ref, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(norm.weight.grad.cpu().double(), dw_ref, rtol=1e-4, atol=1e-4)
    assert x.grad.dtype == torch.float32 and norm.weight.grad.dtype == torch.float32


def test_reference_self_test_fused_rmsnorm_down():
    # the reference's own kernel test: shape, inputs ~ randn bf16 and its tolerances
    from transformer_amd import fused_rmsnorm_down_proj
    g = torch.Generator().manual_seed(42)
    M, K, N = 512, 1792, 384
    x = randn_bf16((M, K), g)
    w_norm = randn_bf16((K,), g)
    w_down = randn_bf16((K, N), g)
    expected = O.rmsnorm_down_proj(x, w_norm, w_down, 1e-6)
    actual = fused_rmsnorm_down_proj(x.cuda(), w_norm.cuda(), w_down.cuda(), 1e-6).cpu()
    m = O.robust_diff(expected, actual)
    assert m["mean"] < 1e-3 and m["p99"] < 0.1, m
    # The reference's `max < 0.5` is below one bf16 ulp for |y| >= 64 (|y| has std ~42 here),
    # so a single output whose fp32 sum lands on the other side of a rounding boundary (a
    # different accumulation order than the CPU's) reaches it; bound each element by one
    # ulp of its expected value instead (at least the ulp of 1.0: outputs near zero come
    # from cancelling sums of terms of size ~1, whose fp32 error is absolute).
    e = expected.float()
    ulp = torch.exp2(torch.floor(torch.log2(e.abs().clamp_min(1.0))) - 7)
    assert ((actual.float() - e).abs() <= ulp).all(), m
    assert m["max"] <= 0.5, m


def test_rmsnorm_config1_shape_sampled_rows(ops):
    # the full norm1 input at B=12, T=2048, d_model=2048; rows sampled for the fp64 check
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(12 * 2048, 2048, generator=g, device="cuda").to(torch.bfloat16)
    w = torch.randn(2048, generator=g, device="cuda")
    y, r = ops.rmsnorm(x, w, 1e-6)
    rows = torch.randint(0, x.size(0), (64,), generator=torch.Generator().manual_seed(1))
    ref = O.rms_norm(x[rows].cpu().double(), w.cpu().double(), 1e-6)
    _bf16_ulp_close(y[rows].cpu(), ref, "config-1 rows")
    assert torch.isfinite(y.float()).all()


@pytest.mark.parametrize("T", [64, 1024])
def test_mla_down_projection_one_gemm_matches_separate_linears(T):
    # T = 1024 (2048 rows) takes the split form: N = 2624 as 2560 + 64 columns
    from transformer_amd import MLA, ModelArgs
    import transformer_amd.mla as M
    args = ModelArgs.mla_baseline(max_seq_len=256)
    m = MLA(args).cuda()
    g = torch.Generator(device="cuda").manual_seed(4)
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn(p.shape, generator=g, device="cuda") * 0.02)
    x = torch.randn(2, T, args.d_model, generator=g, device="cuda")
    assert M._split_pays(2 * T, 2624) == (T == 1024)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        parts = m._down_proj(x)
        refs = (m.q_down(x), m.qk_rope(x), m.kv_down(x))
        again = m._down_proj(x)  # the kept concatenation
    for got, ref, name in zip(parts, refs, ("q_down", "qk_rope", "kv_down")):
        assert got.shape == ref.shape, name
        check_close(got.float(), ref.float().cpu(), name, max_abs=1e-2, mean_abs=1e-4)
    for a, b in zip(parts, again):
        assert torch.equal(a, b)
    # an in-place weight update is seen by the next call
    with torch.no_grad():
        m.kv_down.weight.mul_(2.0)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            kv2 = m._down_proj(x)[2]
    check_close(kv2.float(), 2 * parts[2].float().cpu(), "kv_down after update", max_abs=1e-2, mean_abs=1e-4)


def test_rmsnorm_module_under_torch_compile_matches_eager():
    from transformer_amd import RMSNorm
    g = torch.Generator().manual_seed(12)
    norm = RMSNorm(256).cuda()
    with torch.no_grad():
        norm.weight.copy_(torch.randn(256, generator=g))
    x = torch.randn(3, 17, 256, generator=g).cuda().requires_grad_(True)
    cn = torch.compile(norm, fullgraph=False)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        yc = cn(x)
    yc.float().sum().backward()
    gx, gw = x.grad.clone(), norm.weight.grad.clone()
    x.grad = norm.weight.grad = None
    with torch.autocast("cuda", dtype=torch.bfloat16):
        ye = norm(x)
    ye.float().sum().backward()
    assert torch.equal(yc, ye)
    assert torch.equal(gx, x.grad) and torch.equal(gw, norm.weight.grad)


@pytest.mark.parametrize("M,K", [(7, 1792), (130, 4096), (2049, 512)])
def test_rmsnorm_fp32_output_outside_autocast(ops, M, K):
    # an fp32 module outside autocast gets the reference's fp32 norm (transformer.py:26-27),
    # not a bf16-rounded one; the backward reads an fp32 dy
    from transformer_amd import RMSNorm
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g) * 3
    w = torch.randn(K, generator=g)
    y, r = ops.rmsnorm(x.cuda(), w.cuda(), 1e-6, True)
    assert y.dtype == torch.float32
    ref = O.rms_norm(x.double(), w.double(), 1e-6)
    torch.testing.assert_close(y.cpu().double(), ref, rtol=1e-5, atol=1e-6)
    norm = RMSNorm(K).cuda()
    with torch.no_grad():
        norm.weight.copy_(w)
    xg = x.cuda().requires_grad_(True)
    yy = norm(xg)
    assert yy.dtype == torch.float32
    torch.testing.assert_close(yy.detach().cpu().double(), ref, rtol=1e-5, atol=1e-6)
    dy = torch.randn(M, K, generator=g)
    yy.backward(dy.cuda())
    dx_ref, dw_ref = O.rms_norm_bwd(x, w, dy, 1e-6)
    torch.testing.assert_close(xg.grad.cpu().double(), dx_ref, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(norm.weight.grad.cpu().double(), dw_ref, rtol=1e-4, atol=1e-4)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        assert norm(x.cuda()).dtype == torch.bfloat16  # what the down-projections read under autocast


def test_mla_down_projection_with_frozen_weights_and_input_grad():
    # autograd on, weights frozen, the input needing its gradient: the one-product form (the split
    # form writes into an output buffer, which autograd does not follow)
    from transformer_amd import MLA, ModelArgs
    args = ModelArgs.mla_baseline(max_seq_len=256)
    m = MLA(args).cuda().to(torch.bfloat16)
    for p in m.parameters():
        p.requires_grad_(False)
    x = torch.randn(2, 1024, args.d_model, device="cuda").to(torch.bfloat16).requires_grad_(True)
    q_low, qk_pos, kv_new = m._down_proj(x)
    (q_low.float().sum() + qk_pos.float().sum() + kv_new.float().sum()).backward()
    assert x.grad is not None and torch.isfinite(x.grad.float()).all()


def test_mla_down_projection_split_form_trains_like_one_product(monkeypatch):
    # autograd on under autocast, 2048 rows: the split forward (an autograd Function) against the
    # one-product form: outputs within one bf16 rounding, gradients of x and of the three weights
    # equal to the one product's (the backward is the same single products)
    from transformer_amd import MLA, ModelArgs
    import transformer_amd.mla as M
    args = ModelArgs.mla_baseline(max_seq_len=256)
    m = MLA(args).cuda()
    g = torch.Generator(device="cuda").manual_seed(9)
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn(p.shape, generator=g, device="cuda") * 0.02)
    x0 = torch.randn(2, 1024, args.d_model, generator=g, device="cuda")
    dys = [torch.randn(2, 1024, n, generator=g, device="cuda") for n in (1024, 1088, 512)]

    def run(split):
        monkeypatch.setattr(M, "_split_pays", lambda rows, n: split)
        m.zero_grad(set_to_none=True)
        x = x0.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            outs = m._down_proj(x)
        sum((o.float() * d).sum() for o, d in zip(outs, dys)).backward()
        return [o.detach().float() for o in outs], x.grad, [w.grad.clone() for w in
                                                            (m.q_down.weight, m.qk_rope.weight, m.kv_down.weight)]

    o1, gx1, gw1 = run(True)
    o0, gx0, gw0 = run(False)
    for a, b in zip(o1, o0):
        assert (a - b).abs().max().item() <= 2 ** -7 * b.abs().max().item()
    check_close(gx1.float(), gx0.float().cpu(), "dx", max_abs=1e-2, mean_abs=1e-4)
    for a, b, name in zip(gw1, gw0, ("q_down", "qk_rope", "kv_down")):
        check_close(a.float(), b.float().cpu(), f"d {name}", max_abs=1e-2, mean_abs=1e-4)
