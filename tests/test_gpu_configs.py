"""GPU parity at the benchmark configurations themselves (benchmark configs 0, 3 and 4), each
launched at its full shape and layout and checked against the fp64 oracle.

  config 0: the block's norm1 (RMSNorm, weight 1) and the MLA module in fp32, B=1, T=512,
            d_model 2048, seed 0 (transformer.py:16-27, :202-316, :338);
  config 3: the causal prefill at B=1, T=16384, 16 heads, shared k_rope (transformer.py:314);
  config 4: the attention backward at B=4, T=4096, 16 heads, shared k_rope -- the layout
            bench.py times, whose dk_rope is the sum over the 16 query heads.

Tolerance: max-abs 2e-2 and mean-abs 2e-3 against the fp64 oracle for outputs
of order one (config 0's layer output has max |y| ~ 1.5; attention outputs are averages of
N(0,1) rows), LSE within 1e-3, softmax row sums recomputed from the kernel's LSE within 1e-3.
Gradients use the same bound scaled by max(1, rms(ref)), as tests/test_gpu_backward.py.
"""
import math

import pytest
import torch

from oracle import mla_oracle as O
from tests.gpu_util import ROWSUM_TOL, check_close, randn_bf16, rowsum_from_lse
from tests.test_gpu_backward import check_grad, oracle_grads
from tests.test_gpu_prefill import make_inputs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import transformer_amd  # noqa: F401
    return torch.ops.mla_mi355x


def test_config0_fp32_norm_and_module_vs_oracle():
    from transformer_amd import MLA, ModelArgs, RMSNorm
    args = ModelArgs.mla_baseline(max_seq_len=512)
    dims = O.MLADims(max_seq_len=512)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 512, args.d_model, generator=g)          # hidden ~ N(0, 1), drawn first
    w = O.init_weights(dims, g)                                  # then the weights, registration order
    m = MLA(args)
    m.load_state_dict(w, strict=True)
    norm = RMSNorm(args.d_model, eps=1e-6)                        # weight = 1
    m, norm = m.cuda(), norm.cuda()
    with torch.no_grad():
        xn = norm(x.cuda())
        assert xn.dtype == torch.float32  # the fp32 norm output, as the reference's outside autocast
        y, cache = m(xn)                  # training branch (transformer.py:306-316)
        y_c, c = m(xn, None, True)        # absorbed branch for T > 1 (transformer.py:249-300)
    assert cache is None and y.dtype == torch.float32
    xo = O.rms_norm(x.double(), torch.ones(args.d_model, dtype=torch.float64), 1e-6)
    check_close(xn.double(), xo, "norm1 (fp32)", max_abs=1e-5, mean_abs=1e-6)
    yo, _ = O.mla_forward(w, xo, dims)
    yo_c, co = O.mla_forward(w, xo, dims, use_cache=True)
    check_close(y.double(), yo, "config 0 y (train branch)")
    check_close(y_c.double(), yo_c, "config 0 y (cache branch)")
    assert c["seq_len"] == co["seq_len"] == 512
    check_close(c["latent"].double(), co["latent"], "config 0 cache latent", max_abs=1e-3, mean_abs=1e-4)


def test_config3_long_prefill_sampled_rows(ops):
    B, T, H = 1, 16384, 16
    inp = make_inputs(B, T, T, H, 1, 128, seed=3)
    scale = 1 / math.sqrt(192)
    d = {k: v.cuda() for k, v in inp.items()}
    o, lse = ops.prefill_fwd(d["q_nope"], d["q_rope"], d["k_nope"], d["k_rope"], d["v"], scale, True, 0)
    torch.cuda.synchronize()
    o, lse = o.cpu(), lse.cpu()
    del d
    q = torch.cat([inp["q_nope"], inp["q_rope"]], -1)[0]  # [T, H, 192]
    kr = inp["k_rope"][0, :, 0]
    blocks = [(0, 64), (5000, 5064), (8190, 8260), (16320, 16384)]
    for h in (0, 7, 15):
        k = torch.cat([inp["k_nope"][0, :, h], kr], -1).double()
        v = inp["v"][0, :, h].double()
        for i0, i1 in blocks:
            ro, rl = O.attention(q[i0:i1, h].double(), k[:i1], v[:i1], scale, True, i0)
            check_close(o[0, i0:i1, h].double(), ro, f"O[h={h}, rows {i0}:{i1}]")
            torch.testing.assert_close(lse[0, h, i0:i1].double(), rl, rtol=0, atol=1e-3)
        rows = [0, 5063, 8191, 16383]
        sums = rowsum_from_lse(q[:, h], k, lse[0, h], scale, True, 0, rows)
        assert max(abs(s - 1) for s in sums) <= ROWSUM_TOL, (h, sums)


def test_config4_backward_bench_layout(ops):
    # B=4, T=4096, H=16 with one k_rope head shared by all query heads: the stored-dS path with
    # its ~1.1 GB dS workspace and the fixed-order sum of dk_rope over the heads
    B, T, H = 4, 4096, 16
    inp = make_inputs(B, T, T, H, 1, 128, seed=40)
    do = randn_bf16((B, T, H, 128), torch.Generator().manual_seed(41))
    scale = 1 / math.sqrt(192)
    d = {k: v.cuda() for k, v in inp.items()}
    o, lse = ops.prefill_fwd(d["q_nope"], d["q_rope"], d["k_nope"], d["k_rope"], d["v"], scale, True, 0)
    grads = ops.prefill_bwd(do.cuda(), d["q_nope"], d["q_rope"], d["k_nope"], d["k_rope"], d["v"], o, lse, scale,
                            True, 0)
    torch.cuda.synchronize()
    got = {n: t.cpu() for n, t in zip(("dq_nope", "dq_rope", "dk_nope", "dk_rope", "dv"), grads)}
    del d, o, lse, grads
    assert tuple(got["dk_rope"].shape) == (B, T, 1, 64)
    # every gradient of two sampled (b, h) pairs against the per-head oracle
    for b, h in ((1, 3), (3, 12)):
        sub = {k: v[b:b + 1, :, h:h + 1] if k != "k_rope" else v[b:b + 1] for k, v in inp.items()}
        ref = oracle_grads(sub, do[b:b + 1, :, h:h + 1], scale, True, 0)
        for name in ("dq_nope", "dq_rope", "dk_nope", "dv"):
            check_grad(got[name][b:b + 1, :, h:h + 1], ref[name], f"{name}[b={b},h={h}]")
    # dk_rope of one sequence: the sum over all 16 heads of each head's rope gradient
    b = 2
    acc = torch.zeros(1, T, 1, 64, dtype=torch.float64)
    for h in range(H):
        sub = {k: v[b:b + 1, :, h:h + 1] if k != "k_rope" else v[b:b + 1] for k, v in inp.items()}
        acc += oracle_grads(sub, do[b:b + 1, :, h:h + 1], scale, True, 0)["dk_rope"]
        print(f"dk_rope oracle: head {h} done", flush=True)
    check_grad(got["dk_rope"][b:b + 1], acc, f"dk_rope[b={b}] (sum over {H} heads)")
