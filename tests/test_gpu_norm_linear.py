"""GPU parity of mla_norm_linear, RMSNorm fused into the down-projection (transformer.py:26-27
as norm1, :338, feeding :208-213; the reference's fused kernel fused_mla_triton_kernels.py:105-274),
against the oracle's rmsnorm_down_proj: bf16(bf16(norm(x) * w_norm) @ w_down) in fp64.

Bounds: r within 2e-6 (relative) of the fp64 formula; given the kernel's r, the normalised rows
bf16((x * r) * w_norm) are exact fp32 arithmetic, so each output is within one bf16 ulp (at least
the ulp of 1.0, for outputs that cancel) of the fp64 product of those rows; against the oracle
itself the reference's own self-test tolerances hold (mean < 1e-3, p99 < 0.1, max < 0.5: a last
bit of r that differs from the oracle's division can flip one normalised element, which moves a
whole output row by ulp(xn) |W|)."""
import pytest
import torch

from oracle import mla_oracle as O
from tests.gpu_util import randn_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import transformer_amd  # noqa: F401
    return torch.ops.mla_mi355x


def within_one_ulp(actual, expected, what):
    e = expected.float()
    ulp = torch.exp2(torch.floor(torch.log2(e.abs().clamp_min(1.0))) - 7)
    d = (actual.float() - e).abs()
    assert torch.isfinite(actual.float()).all(), what
    assert (d <= ulp).all(), f"{what}: {(d > ulp).sum().item()} outputs beyond one ulp, max excess {(d - ulp).max().item():.3g}"


def expected_from_r(x, w_norm, w, r):
    """fp64 product of the normalised rows the kernel forms from its own r (rows of x [M, K],
    w [N, K] nn.Linear layout); the rounding of (x * r) * w_norm is fp32 on both sides."""
    xn = ((x.float() * r.cpu().float()[:, None]) * w_norm.cpu().float()).to(torch.bfloat16)
    return xn.double() @ w.double().t()


def check_r(r, x, eps):
    r_ref = 1.0 / torch.sqrt(x.double().pow(2).mean(-1) + eps)
    torch.testing.assert_close(r.cpu().double(), r_ref, rtol=2e-6, atol=0)


def test_norm_linear_reference_self_test(ops):
    # the reference's own kernel test (fused_mla_triton_kernels.py:800-830): seed 42, M = 512,
    # K = 1792, N = 384, inputs ~ randn bf16; its mean < 1e-3, p99 < 0.1 and max < 0.5
    g = torch.Generator().manual_seed(42)
    M, K, N = 512, 1792, 384
    x = randn_bf16((M, K), g)
    w_norm = randn_bf16((K,), g)
    w_down = randn_bf16((K, N), g)
    expected = O.rmsnorm_down_proj(x, w_norm, w_down, 1e-6)
    y, r = ops.norm_linear(x.cuda(), w_down.t().contiguous().cuda(), w_norm.cuda(), 1e-6)
    m = O.robust_diff(expected, y.cpu())
    assert m["mean"] < 1e-3 and m["p99"] < 0.1 and m["max"] <= 0.5, m
    check_r(r, x, 1e-6)
    within_one_ulp(y.cpu(), expected_from_r(x, w_norm, w_down.t(), r), "self-test shape")


@pytest.mark.parametrize("M,N,K", [(33, 4, 32), (300, 100, 96), (256, 256, 64), (257, 260, 2048), (1000, 2624, 2048),
                                   (40, 520, 4096)])
def test_norm_linear_ragged_shapes(ops, M, N, K):
    print(f"case M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M + N + K)
    x = randn_bf16((M, K), g)
    w = randn_bf16((N, K), g, 0.05)
    w_norm = torch.rand(K, generator=g) + 0.5
    y, r = ops.norm_linear(x.cuda(), w.cuda(), w_norm.cuda(), 1e-6)
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    check_r(r, x, 1e-6)
    within_one_ulp(y.cpu(), expected_from_r(x, w_norm, w, r), f"M={M} N={N} K={K}")


def test_norm_linear_config1_rows_and_the_unfused_path(ops):
    # config 1's norm1 input (B=12, T=2048, d_model 2048) through the three down-projections
    # (N = 1024 + 17 * 64 + 512): sampled rows against the oracle; the whole output against the
    # unfused path (the RMSNorm kernel's bf16 rows, then the same product in fp32 on the GPU)
    g = torch.Generator(device="cuda").manual_seed(21)
    M, K, N = 12 * 2048, 2048, 2624
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    w_norm = torch.rand(K, generator=g, device="cuda") + 0.5
    y, r = ops.norm_linear(x, w, w_norm, 1e-6)
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(22))[:48]
    check_r(r[rows], x[rows].cpu(), 1e-6)
    within_one_ulp(y[rows].cpu(), expected_from_r(x[rows].cpu(), w_norm, w.cpu(), r[rows]), "config 1 rows")
    m = O.robust_diff(O.rmsnorm_down_proj(x[rows].cpu(), w_norm.cpu(), w.t().cpu(), 1e-6), y[rows].cpu())
    assert m["mean"] < 1e-3 and m["p99"] < 0.1 and m["max"] <= 0.5, m
    # the unfused path: the RMSNorm kernel's bf16 rows, then the product in fp32 on the GPU
    xn, r2 = ops.rmsnorm(x, w_norm, 1e-6)
    torch.testing.assert_close(r, r2, rtol=2e-6, atol=0)
    ref = (xn.float() @ w.float().t()).to(torch.bfloat16)
    m = O.robust_diff(ref.float().cpu(), y.float().cpu())
    assert m["mean"] < 1e-4 and m["max"] <= 0.05, m


def test_norm_linear_strided_rows_batched_and_deterministic(ops):
    g = torch.Generator().manual_seed(23)
    buf = randn_bf16((2, 70, 520), g)
    x = buf[..., 8:8 + 512]  # rows of stride 520, batched leading dims
    w = randn_bf16((96, 512), g, 0.05)
    w_norm = torch.rand(512, generator=g) + 0.5
    y, r = ops.norm_linear(x.cuda(), w.cuda(), w_norm.cuda(), 1e-5)
    assert y.shape == (2, 70, 96) and r.shape == (2, 70)
    check_r(r.reshape(-1), x.reshape(-1, 512), 1e-5)
    within_one_ulp(y.cpu().reshape(-1, 96), expected_from_r(x.reshape(-1, 512), w_norm, w, r.reshape(-1)), "strided")
    y2, _ = ops.norm_linear(x.cuda(), w.cuda(), w_norm.cuda(), 1e-5)
    assert torch.equal(y, y2)


def test_norm_linear_rejects_bad_shapes(ops):
    x = torch.zeros(4, 48, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        ops.norm_linear(x, torch.zeros(8, 48, dtype=torch.bfloat16, device="cuda"), torch.ones(48, device="cuda"), 1e-6)
    x = torch.zeros(4, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        ops.norm_linear(x, torch.zeros(6, 64, dtype=torch.bfloat16, device="cuda"), torch.ones(64, device="cuda"), 1e-6)
    with pytest.raises(TypeError):
        ops.norm_linear(x.float(), torch.zeros(8, 64, dtype=torch.bfloat16, device="cuda"), torch.ones(64, device="cuda"),
                        1e-6)
