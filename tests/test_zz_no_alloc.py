"""GPU test of mla_decode_static, the decode entry point that allocates nothing (its split
partials live in a static device array), called through the C ABI: two calls in a row, the
second on a smaller input, each checked against mla_decode with a caller workspace on the
same arguments (the same kernels and split layout, so bitwise equal) and against the fp64
oracle's absorbed decode (transformer.py:249-286) at the path's bf16 tolerance (max-abs 2e-2, mean-abs 2e-3)."""
import ctypes
import math

import pytest
import torch

from oracle import mla_oracle as O
from tests.gpu_util import check_close, randn_bf16

pytestmark = pytest.mark.gpu


def _inputs(B, L, H, DL, seed):
    g = torch.Generator().manual_seed(seed)
    return (randn_bf16((B, H, DL), g, 0.3), randn_bf16((B, H, 64), g, 0.3), randn_bf16((B, L, DL), g),
            randn_bf16((B, 1, L, 64), g))


def _call(entry, q_lat, q_rope, c_kv, k_rope, seq_lens, scale, workspace):
    from transformer_amd import _lib, kernels
    B, H, DL = q_lat.shape
    ctx = torch.full((B, H, DL), float("nan"), dtype=torch.bfloat16, device="cuda")
    lse = torch.full((B, H), float("nan"), dtype=torch.float32, device="cuda")
    args, keep = kernels._decode_args(entry, q_lat, q_rope, c_kv, k_rope, seq_lens, scale, 0, ctx, lse)
    ws = None
    if workspace:
        n = int(_lib.entry("mla_decode_workspace_bytes")(ctypes.byref(args)))
        ws = torch.empty(max(n, 1), dtype=torch.uint8, device="cuda")
        args.workspace, args.workspace_bytes = ws.data_ptr(), n
    rc = _lib.entry(entry)(ctypes.byref(args), torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, entry)
    torch.cuda.synchronize()
    return ctx.cpu(), lse.cpu(), int(_lib.entry("mla_decode_workspace_bytes")(ctypes.byref(args)))


@pytest.mark.parametrize("B,L,H,DL,lens", [(32, 4096, 16, 512, None), (3, 300, 16, 512, [300, 1, 177]),
                                           (1, 20000, 16, 512, None)])
def test_decode_static_matches_decode_twice(B, L, H, DL, lens):
    import transformer_amd  # noqa: F401
    from transformer_amd import _lib
    print(f"case B={B} L={L} H={H} DL={DL} lens={lens}", flush=True)
    scale = 1 / math.sqrt(192)
    # two calls in a row, the second on a smaller input: the array keeps the first call's partials
    for rep, (b, l) in enumerate(((B, L), (max(1, B // 2), max(2, L // 3)))):
        q_lat, q_rope, c_kv, k_rope = _inputs(b, l, H, DL, seed=B * 13 + L + rep)
        sl = None if lens is None else torch.tensor([min(x, l) for x in lens[:b]], dtype=torch.int32)
        dev = [t.cuda() for t in (q_lat, q_rope, c_kv, k_rope)]
        sld = None if sl is None else sl.cuda()
        ctx_s, lse_s, need = _call("mla_decode_static", *dev, sld, scale, workspace=False)
        ctx_w, lse_w, _ = _call("mla_decode", *dev, sld, scale, workspace=True)
        assert need <= _lib.MLA_DECODE_STATIC_SCRATCH_BYTES
        assert torch.equal(ctx_s, ctx_w) and torch.equal(lse_s, lse_w), f"call {rep}: differs from mla_decode"
        ref_ctx, ref_lse = O.absorbed_decode(q_lat.double().unsqueeze(2), q_rope.double().unsqueeze(2),
                                             c_kv.double(), k_rope.double(), scale,
                                             seq_lens=None if sl is None else sl.tolist())
        ref_ctx, ref_lse = ref_ctx.squeeze(2), ref_lse.squeeze(2)
        valid = torch.ones(b, dtype=torch.bool) if sl is None else sl > 0
        check_close(ctx_s[valid].double(), ref_ctx[valid], f"ctx (static, call {rep})")
        torch.testing.assert_close(lse_s[valid].double(), ref_lse[valid], rtol=0, atol=1e-3)

