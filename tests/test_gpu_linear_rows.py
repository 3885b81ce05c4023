"""GPU parity of mla_linear_rows, the few-row products of the decode step (transformer.py:208-213
q_down / qk_rope / kv_down, :208 q_up, :252-254 the W_UK absorption, :300 o_proj at T == 1),
against an fp64 product of the same bf16 inputs.

Bound: the kernel accumulates in fp32 and rounds once to bf16, so every element is within one
bf16 ulp (2^-8 relative) of the fp64 value plus the fp32 accumulation error of K products
(K 2^-24 max|x| max|w| per term, taken as an absolute floor)."""
import pytest
import torch

from tests.gpu_util import randn_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import transformer_amd  # noqa: F401
    return torch.ops.mla_mi355x


def check_rows(y, ref, K, xmax, wmax, what):
    y = y.cpu().double()
    bound = ref.abs() * 2.0 ** -8 + K * 2.0 ** -22 * xmax * wmax
    err = (y - ref).abs()
    assert torch.isfinite(y).all(), what
    assert (err <= bound).all(), f"{what}: max excess {(err - bound).max().item():.3e}"


@pytest.mark.parametrize("M,N,K", [(1, 4, 128), (32, 2624, 2048), (32, 2048, 1024), (32, 2048, 2048), (7, 100, 384),
                                   (17, 64, 640), (64, 512, 2048), (100, 48, 256), (32, 36, 4096)])
def test_linear_rows_matches_fp64(ops, M, N, K):
    print(f"case M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M * 131 + N + K)
    x = randn_bf16((M, K), g)
    w = randn_bf16((N, K), g, 0.02)
    y = ops.linear_rows(x.cuda(), w.cuda())
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    ref = x.double() @ w.double().t()
    check_rows(y, ref, K, x.abs().max().item(), w.abs().max().item(), f"M={M} N={N} K={K}")


@pytest.mark.parametrize("M", [16, 17, 32, 33, 64])
def test_linear_rows_waves_with_one_or_two_k_steps(ops, M):
    # K = 128 .. 384 gives each of the four waves one to three k-steps of a 16-step pass: the
    # steps past a wave's count must not reach the MFMA (regression: a lane-masked guard let
    # them run on unloaded registers)
    g = torch.Generator().manual_seed(M)
    for K in (128, 256, 384, 640):
        x = randn_bf16((M, K), g)
        w = randn_bf16((96, K), g, 0.05)
        y = ops.linear_rows(x.cuda(), w.cuda())
        ref = x.double() @ w.double().t()
        check_rows(y, ref, K, x.abs().max().item(), w.abs().max().item(), f"M={M} K={K}")


def test_linear_rows_grouped_absorption_layout(ops):
    # q_lat[b, h] = q_nope[b, h] W_UK[h] with q_nope read in place from q_up's output rows
    # [B, H * dn] and W_UK transposed per head [H, DL, dn] (transformer.py:252-254)
    g = torch.Generator().manual_seed(5)
    B, H, dn, DL = 32, 16, 128, 512
    q_up_out = randn_bf16((B, H * dn), g)
    w_uk = randn_bf16((H, dn, DL), g, 0.05)  # k_up.weight.view(H, dn, DL)
    y = ops.linear_rows(q_up_out.cuda().view(B, H, dn), w_uk.cuda().transpose(1, 2).contiguous())
    assert y.shape == (B, H, DL)
    ref = torch.einsum("bhd,hdc->bhc", q_up_out.double().view(B, H, dn), w_uk.double())
    check_rows(y, ref, dn, q_up_out.abs().max().item(), w_uk.abs().max().item(), "grouped absorption")


def test_linear_rows_strided_rows_and_bad_shapes(ops):
    g = torch.Generator().manual_seed(6)
    buf = randn_bf16((32, 3000), g)
    x = buf.cuda()[:, 8:8 + 1024]  # rows of stride 3000, 16-byte aligned start
    w = randn_bf16((256, 1024), g, 0.02).cuda()
    y = ops.linear_rows(x, w)
    ref = buf[:, 8:8 + 1024].double() @ w.cpu().double().t()
    check_rows(y, ref, 1024, buf.abs().max().item(), w.abs().max().item(), "strided x")
    with pytest.raises(ValueError):
        ops.linear_rows(x[:, :1000], w[:, :1000])  # K not a multiple of 128
    with pytest.raises(TypeError):
        ops.linear_rows(x.float(), w)


def test_linear_rows_is_deterministic(ops):
    g = torch.Generator().manual_seed(7)
    x, w = randn_bf16((32, 2048), g).cuda(), randn_bf16((2624, 2048), g, 0.02).cuda()
    assert torch.equal(ops.linear_rows(x, w), ops.linear_rows(x, w))


@pytest.mark.parametrize("B,pos_dev,C", [(32, True, 4096), (1, True, 1536), (4, False, 300), (48, True, 1000),
                                         (0, True, 64)])
def test_linear_rows_rope_append_equals_the_two_ops(ops, B, pos_dev, C):
    # the decode step's q_up product beside the RoPE + cache append (transformer.py:208, :215-244)
    # in one launch: every output and every cache write bit for bit the two ops' (B = 0: nothing
    # to multiply or append, and no launch fails)
    print(f"case linear_rows_rope_append B={B} pos_dev={pos_dev} C={C}", flush=True)
    from oracle import mla_oracle as O
    H, Hr, DL, K, N = 16, 1, 512, 1024, 2048
    g = torch.Generator().manual_seed(B * 7 + C)
    down = randn_bf16((B, 1024 + (H + Hr) * 64 + DL), g).cuda()  # the down-projections' output rows
    x, qk, c_new = down[:, :1024], down[:, 1024:1024 + (H + Hr) * 64], down[:, 1024 + (H + Hr) * 64:]
    w = randn_bf16((N, K), g, 0.02).cuda()
    cos, sin = (t.to(torch.bfloat16).cuda() for t in O.rope_tables(64, 8192))
    caches = []
    for _ in range(2):
        lat = randn_bf16((B, C, DL), g).cuda()
        kr = randn_bf16((B, Hr, C, 64), g).cuda()
        caches.append((lat, kr, torch.zeros(B, dtype=torch.int32, device="cuda"),
                       torch.zeros(1, dtype=torch.int64, device="cuda")))
    caches[1] = tuple(t.clone() for t in caches[0])
    L0 = C // 2 + 3
    pos = torch.full((1,), L0, dtype=torch.int64, device="cuda") if pos_dev else None
    off = 0 if pos_dev else L0
    qk4, c3 = qk.reshape(B, 1, H + Hr, 64), c_new.reshape(B, 1, DL)
    lat, kr, sl, pn = caches[0]
    y_ref = ops.linear_rows(x, w)
    q_ref = ops.rope_append(qk4, c3, lat, kr, cos, sin, pos, sl, off, H, pn)
    lat2, kr2, sl2, pn2 = caches[1]
    y, q = ops.linear_rows_rope_append(x, w, qk4, c3, lat2, kr2, cos, sin, pos, sl2, off, H, pn2)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref) and torch.equal(q, q_ref)
    assert torch.equal(lat2, lat) and torch.equal(kr2, kr) and torch.equal(sl2, sl) and torch.equal(pn2, pn)
    if B:
        assert (sl2 == L0 + 1).all() and pn2.item() == L0 + 1
        assert torch.equal(lat2[:, L0], c_new)
