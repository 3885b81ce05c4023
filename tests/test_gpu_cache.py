"""GPU tests of the module's preallocated KV-cache (autograd off) against its torch.cat
path (autograd on, the reference's growth at transformer.py:215-218,241-244): the same
outputs and cache contents, decode steps bitwise, and branching from an older dict.

These compare the eager kernels, so the module's recorded one-token step is switched off
here: it splits each sequence's own length at run time, which rounds the split merge
differently from the host's split at small batches (its own tests: test_gpu_auto_graph.py)."""
import pytest
import torch

import transformer_amd.mla as M
from tests.test_gpu_module import _baseline_module, rel_check

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _eager_steps(monkeypatch):
    monkeypatch.setattr(M, "AUTO_GRAPH", False)


def _steps(m, x, splits, grad):
    """run x in the given token splits through the cached path; returns outputs and caches"""
    outs, caches, c = [], [], None
    ctx = torch.enable_grad() if grad else torch.no_grad()
    with ctx, torch.autocast("cuda", dtype=torch.bfloat16):
        t = 0
        for n in splits:
            y, c = m(x[:, t:t + n], c, True)
            outs.append(y.detach().float())
            caches.append({k: (v.detach().clone() if torch.is_tensor(v) else v) for k, v in c.items()})
            t += n
    return outs, caches, c


def test_preallocated_cache_matches_cat_path():
    m, args = _baseline_module(seed=11)
    x = torch.randn(2, 300, args.d_model, generator=torch.Generator().manual_seed(12)).cuda()
    splits = [200, 1, 1, 1, 60, 1, 1, 36]  # prefill, decode, chunk, decode, chunk past the first capacity
    got, got_c, last = _steps(m, x, splits, grad=False)
    ref, ref_c, _ = _steps(m, x, splits, grad=True)
    for i, (a, b, n) in enumerate(zip(got, ref, splits)):
        if n == 1:
            assert torch.equal(a, b), f"decode step {i}"
        else:
            rel_check(a, b, f"chunk step {i}", rmax=1e-2, rmean=1e-3)
    for i, (a, b) in enumerate(zip(got_c, ref_c)):
        assert a["seq_len"] == b["seq_len"]
        for k in ("latent", "k_rope"):
            assert a[k].shape == b[k].shape and torch.equal(a[k], b[k]), f"cache {k} after step {i}"
    # the last cache is a view of buffers with spare room (no O(L) copy on the next append)
    assert last["latent"].stride(0) > last["latent"].size(1) * last["latent"].size(2)


def test_branching_from_an_older_cache_dict():
    m, args = _baseline_module(seed=13)
    g = torch.Generator().manual_seed(14)
    x = torch.randn(1, 64, args.d_model, generator=g).cuda()
    xa = torch.randn(1, 1, args.d_model, generator=g).cuda()
    xb = torch.randn(1, 1, args.d_model, generator=g).cuda()
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        _, c = m(x, None, True)
        ya, ca = m(xa, c, True)
        saved = ca["latent"].clone(), ca["k_rope"].clone()
        yb, cb = m(xb, c, True)  # branch from the older dict
        assert torch.equal(ca["latent"], saved[0]) and torch.equal(ca["k_rope"], saved[1])
        ya2, _ = m(xa, c, True)
    with torch.enable_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        _, cr = m(x, None, True)
        yb_ref, cb_ref = m(xb, cr, True)
    assert torch.equal(ya2, ya)
    assert torch.equal(yb.float(), yb_ref.detach().float())
    assert torch.equal(cb["latent"], cb_ref["latent"]) and torch.equal(cb["k_rope"], cb_ref["k_rope"])


def test_inference_mode_cache():
    m, args = _baseline_module(seed=15)
    x = torch.randn(2, 40, args.d_model, generator=torch.Generator().manual_seed(16)).cuda()
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        full, _ = m(x)
        y0, c = m(x[:, :38], None, True)
        y1, c = m(x[:, 38:39], c, True)
        y2, c = m(x[:, 39:], c, True)
    rel_check(torch.cat([y0, y1, y2], 1).float(), full.float(), "inference-mode cached vs full")
    assert c["seq_len"] == 40


def test_rope_append_path_is_bitwise_equal_to_rope_and_copies():
    # the cache path with RoPE writing the new slots itself (rope_append) against RoPE then two
    # copies into the same preallocated buffers: identical outputs and caches, bit for bit
    m, args = _baseline_module(seed=21)
    x = torch.randn(2, 140, args.d_model, generator=torch.Generator().manual_seed(22)).cuda()
    splits = [100, 1, 1, 30, 1, 7]
    saved = M.ROPE_APPEND
    try:
        M.ROPE_APPEND = True
        a_out, a_c, _ = _steps(m, x, splits, grad=False)
        M.ROPE_APPEND = False
        b_out, b_c, _ = _steps(m, x, splits, grad=False)
    finally:
        M.ROPE_APPEND = saved
    for ya, yb in zip(a_out, b_out):
        assert torch.equal(ya, yb)
    for ca, cb in zip(a_c, b_c):
        assert ca["seq_len"] == cb["seq_len"]
        assert torch.equal(ca["latent"], cb["latent"]) and torch.equal(ca["k_rope"], cb["k_rope"])
