"""The module layer's eager calls (``kernels.eager``: the operators' bodies without the torch
dispatcher, where nothing needs it) against the registered operators on the same inputs:
bitwise equal results, and the registered operator (with its autograd formula) taken when an
input needs a gradient."""
import math

import pytest
import torch

from tests.gpu_util import randn_bf16
from transformer_amd import kernels

pytestmark = pytest.mark.gpu

SCALE = 1 / math.sqrt(192)


@pytest.fixture(scope="module")
def ops():
    import transformer_amd  # noqa: F401
    return torch.ops.mla_mi355x


def same(a, b):
    if isinstance(a, (tuple, list)):
        assert len(a) == len(b)
        for x, y in zip(a, b):
            same(x, y)
    else:
        assert torch.equal(a, b)


def test_eager_calls_equal_the_operators(ops):
    print("case eager vs operators", flush=True)
    g = torch.Generator().manual_seed(31)
    e = kernels.eager
    with torch.no_grad():
        x = randn_bf16((2, 40, 17, 64), g).cuda()
        cos = torch.randn(64, 32, generator=g).to(torch.bfloat16).cuda()
        sin = torch.randn(64, 32, generator=g).to(torch.bfloat16).cuda()
        assert not kernels.dispatcher_needed((x, cos, sin, 3, False))
        same(e.rope(x, cos, sin, 3, False), ops.rope(x, cos, sin, 3, False))
        qn, qr, kn, kr, v = (randn_bf16(s, g).cuda() for s in ((2, 70, 4, 128), (2, 70, 4, 64), (2, 70, 4, 128),
                                                                (2, 70, 1, 64), (2, 70, 4, 128)))
        same(e.prefill_fwd(qn, qr, kn, kr, v, SCALE, True, 0), ops.prefill_fwd(qn, qr, kn, kr, v, SCALE, True, 0))
        ql, qrd, c, krd = (randn_bf16(s, g).cuda() for s in ((3, 16, 512), (3, 16, 64), (3, 300, 512), (3, 1, 300, 64)))
        same(e.decode(ql, qrd, c, krd, None, SCALE, 0), ops.decode(ql, qrd, c, krd, None, SCALE, 0))
        xr, w = randn_bf16((5, 256), g).cuda(), randn_bf16((96, 256), g, 0.05).cuda()
        same(e.linear_rows(xr, w), ops.linear_rows(xr, w))
        wn = (torch.rand(256, generator=g) + 0.5).cuda()
        same(e.rmsnorm(xr, wn, 1e-6, False), ops.rmsnorm(xr, wn, 1e-6, False))
        same(e.norm_linear(xr, w, wn, 1e-6), ops.norm_linear(xr, w, wn, 1e-6))
        qc, qcr, cc, kc = (randn_bf16(s, g).cuda() for s in ((1, 8, 16, 512), (1, 8, 16, 64), (1, 108, 512),
                                                              (1, 1, 108, 64)))
        same(e.prefill_cached(qc, qcr, cc, kc, 100, SCALE), ops.prefill_cached(qc, qcr, cc, kc, 100, SCALE))


def test_eager_calls_keep_the_autograd_formulas():
    print("case eager autograd", flush=True)
    g = torch.Generator().manual_seed(32)
    x = randn_bf16((1, 8, 2, 64), g).cuda().requires_grad_()
    cos = torch.randn(16, 32, generator=g).to(torch.bfloat16).cuda()
    sin = torch.randn(16, 32, generator=g).to(torch.bfloat16).cuda()
    assert kernels.dispatcher_needed((x, cos, sin, 0, False))
    y = kernels.eager.rope(x, cos, sin, 0, False)
    assert y.grad_fn is not None
    y.float().sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad.float()).all()
    with torch.no_grad():
        assert not kernels.dispatcher_needed((x, cos, sin, 0, False))
        assert kernels.eager.rope(x, cos, sin, 0, False).grad_fn is None


def test_launch_stream_is_torchs_current_stream():
    x = torch.zeros(4, device="cuda")
    assert kernels._stream(x) == torch.cuda.current_stream(x.device).cuda_stream
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert kernels._stream(x) == side.cuda_stream != torch.cuda.default_stream(x.device).cuda_stream
    torch.cuda.synchronize()
