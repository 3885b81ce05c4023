"""GPU parity of the fused RoPE kernel (mla_rope) against the oracle's apply_rope
(transformer.py:55-60)."""
import pytest
import torch

from oracle import mla_oracle as O
from tests.gpu_util import randn_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import transformer_amd  # noqa: F401
    return torch.ops.mla_mi355x


def _tables(rows=4096):
    cos, sin = O.rope_tables(64, rows, 10000.0)
    return cos, sin


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,T,NH,pos", [(1, 1, 1, 0), (2, 37, 17, 0), (3, 64, 2, 100), (1, 5, 33, 4000)])
def test_rope_matches_oracle(ops, dtype, B, T, NH, pos):
    g = torch.Generator().manual_seed(B * 1000 + T)
    x = randn_bf16((B, T, NH, 64), g).to(dtype)
    cos, sin = _tables()
    y = ops.rope(x.cuda(), cos.cuda(), sin.cuda(), pos, False).cpu()
    c, s = cos[pos:pos + T].double(), sin[pos:pos + T].double()
    ref = O.apply_rope(x.double().transpose(1, 2), c, s).transpose(1, 2)
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-5
    assert (y.double() - ref).abs().max().item() <= tol * max(1.0, ref.abs().max().item())
    if dtype == torch.float32:
        torch.testing.assert_close(y.double(), ref, rtol=1e-5, atol=1e-5)


def test_rope_inverse_roundtrip_and_strided(ops):
    g = torch.Generator().manual_seed(7)
    buf = randn_bf16((2, 19, 5 * 64 + 64), g).float()  # fp32: exact roundtrip check
    x = buf[..., 64:].reshape(2, 19, 5, 64)  # strided view (token stride 384)
    cos, sin = _tables()
    xc = x.cuda()
    y = ops.rope(xc, cos.cuda(), sin.cuda(), 3, False)
    back = ops.rope(y, cos.cuda(), sin.cuda(), 3, True).cpu()
    norm = (cos[3:22].double() ** 2 + sin[3:22].double() ** 2).repeat(1, 2)[None, :, None, :]
    torch.testing.assert_close(back.double() / norm, x.double(), rtol=1e-5, atol=1e-5)


def test_rope_inplace_matches_out_of_place(ops):
    g = torch.Generator().manual_seed(8)
    x = randn_bf16((2, 9, 3, 64), g).cuda()
    cos, sin = (t.cuda() for t in _tables())
    y = ops.rope(x, cos, sin, 11, False)
    ops.rope_(x, cos, sin, 11, False)
    assert torch.equal(x, y)


def test_rope_autograd_is_inverse_rotation(ops):
    g = torch.Generator().manual_seed(9)
    x = randn_bf16((1, 6, 2, 64), g).float().cuda().requires_grad_(True)
    cos, sin = (t.cuda() for t in _tables())
    dy = torch.randn(1, 6, 2, 64, generator=g).cuda()
    ops.rope(x, cos, sin, 0, False).backward(dy)
    ref = ops.rope(dy, cos, sin, 0, True)
    torch.testing.assert_close(x.grad, ref)


def test_rope_rejects_table_overflow(ops):
    x = torch.zeros(1, 4, 1, 64, dtype=torch.bfloat16).cuda()
    cos, sin = (t.cuda() for t in _tables(16))
    with pytest.raises(RuntimeError, match="exceed"):
        ops.rope(x, cos, sin, 14, False)


@pytest.mark.parametrize("B,T,H,Hr,DL,C,pos", [(1, 1, 16, 1, 512, 64, 0), (3, 1, 16, 1, 512, 300, 257),
                                              (2, 5, 14, 14, 384, 40, 30), (4, 2, 4, 1, 64, 9, 7)])
@pytest.mark.parametrize("device_pos", [False, True])
def test_rope_append_matches_rope_and_copies(ops, B, T, H, Hr, DL, C, pos, device_pos):
    print(f"case B={B} T={T} H={H} Hr={Hr} DL={DL} C={C} pos={pos} device_pos={device_pos}", flush=True)
    g = torch.Generator().manual_seed(B * 100 + T * 10 + H)
    cos, sin = _tables(512)
    cos, sin = cos.cuda(), sin.cuda()
    proj = randn_bf16((B, T, 3 * DL), g).cuda()  # the new latent rows as a strided column view
    c_new = proj[..., DL:2 * DL]
    qk = randn_bf16((B, T, H + Hr, 64), g).cuda()
    latent0 = randn_bf16((B, C, DL), g).cuda()
    k0 = randn_bf16((B, Hr, C, 64), g).cuda()
    latent, kc = latent0.clone(), k0.clone()
    seq_lens = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    if device_pos:
        nxt = torch.full((1,), -7, dtype=torch.int64, device="cuda")
        q = ops.rope_append(qk, c_new, latent, kc, cos, sin, torch.tensor([pos], device="cuda"), seq_lens, 0, H, nxt)
        assert int(nxt.item()) == pos + T, "the next position is pos + T"
    else:
        q = ops.rope_append(qk, c_new, latent, kc, cos, sin, None, seq_lens, pos, H, None)
    ref = ops.rope(qk, cos, sin, pos, False)
    assert torch.equal(q, ref[:, :, :H]), "q heads differ from mla_rope"
    assert torch.equal(kc[:, :, pos:pos + T], ref[:, :, H:].transpose(1, 2)), "k heads not written to the cache"
    assert torch.equal(latent[:, pos:pos + T], c_new), "latent rows not copied"
    keep = torch.ones(C, dtype=torch.bool)
    keep[pos:pos + T] = False
    assert torch.equal(latent[:, keep], latent0[:, keep]) and torch.equal(kc[:, :, keep], k0[:, :, keep])
    assert (seq_lens == pos + T).all()


def test_rope_append_skips_a_device_position_past_the_end(ops):
    # a device-side position at the capacity writes nothing (the kernel's own bounds check)
    g = torch.Generator().manual_seed(3)
    cos, sin = _tables(64)
    qk = randn_bf16((2, 1, 5, 64), g).cuda()
    c_new = randn_bf16((2, 1, 64), g).cuda()
    latent = randn_bf16((2, 16, 64), g).cuda()
    kc = randn_bf16((2, 1, 16, 64), g).cuda()
    l0, k0 = latent.clone(), kc.clone()
    ops.rope_append(qk, c_new, latent, kc, cos.cuda(), sin.cuda(), torch.tensor([16], device="cuda"), None, 0, 4, None)
    torch.cuda.synchronize()
    assert torch.equal(latent, l0) and torch.equal(kc, k0)
    with pytest.raises(Exception):  # a host position past the end is refused before any launch
        ops.rope_append(qk, c_new, latent, kc, cos.cuda(), sin.cuda(), None, None, 16, 4, None)
