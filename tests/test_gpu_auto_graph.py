"""GPU tests of the module's recorded one-token step (transformer.py:202-300 with T == 1 and a
cache): with autograd off and bf16 weights, ``MLA.forward`` replays a HIP graph bound to the
cache's own buffers.  Every step is compared with the eager kernels (``AUTO_GRAPH = False``)
from the same starting cache: outputs and caches bit for bit where both split the context
alike (B = 32 at 1024 positions or more), within rounding otherwise; across buffer growth,
a weight change, branching from an older dict and caches used in turn."""
import pytest
import torch

import transformer_amd.mla as M
from tests.test_gpu_module import _baseline_module, rel_check

pytestmark = pytest.mark.gpu


def _bf16_module(seed):
    m, args = _baseline_module(seed=seed)
    return m.to(torch.bfloat16), args


def _cache(B, L, args, seed):
    g = torch.Generator().manual_seed(seed)
    return {"latent": torch.randn(B, L, args.d_latent, generator=g).to(torch.bfloat16).cuda(),
            "k_rope": torch.randn(B, 1, L, 64, generator=g).to(torch.bfloat16).cuda(), "seq_len": L}


def _run(m, c, xs, graph):
    saved = M.AUTO_GRAPH
    M.AUTO_GRAPH = graph
    try:
        ys = []
        with torch.no_grad():
            for x in xs:
                y, c = m(x, c, True)
                ys.append(y)
        return ys, c
    finally:
        M.AUTO_GRAPH = saved


def _same_cache(a, b, what):
    assert a["seq_len"] == b["seq_len"], what
    assert torch.equal(a["latent"], b["latent"]) and torch.equal(a["k_rope"], b["k_rope"]), what


def test_recorded_step_is_bitwise_the_eager_step():
    m, args = _bf16_module(31)
    print("case B=32 L0=1100 N=12", flush=True)
    B, L0, N = 32, 1100, 12
    c0 = _cache(B, L0, args, 32)
    g = torch.Generator().manual_seed(33)
    xs = [torch.randn(B, 1, args.d_model, generator=g).to(torch.bfloat16).cuda() for _ in range(N)]
    ye, ce = _run(m, c0, xs, graph=False)
    yg, cg = _run(m, c0, xs, graph=True)
    st = m.__dict__.get("_graph_state")
    assert st is not None and st["graph"] is not None, "the step was not recorded"
    for i, (a, b) in enumerate(zip(yg, ye)):
        assert torch.equal(a, b), f"step {i}"
    _same_cache(cg, ce, "final cache")
    # outputs are fresh tensors: an earlier step's output survives later replays
    assert yg[0].data_ptr() != yg[1].data_ptr()
    m.release_decode_graph()
    assert "_graph_state" not in m.__dict__


def test_recorded_step_across_growth_weight_change_and_branch():
    m, args = _bf16_module(34)
    B, L0, N = 2, 200, 320  # the store (512 positions) fills and grows during the run
    c0 = _cache(B, L0, args, 35)
    g = torch.Generator().manual_seed(36)
    xs = [torch.randn(B, 1, args.d_model, generator=g).to(torch.bfloat16).cuda() for _ in range(N + 6)]
    print("case growth B=2 L0=200", flush=True)
    ye, ce = _run(m, c0, xs[:N], graph=False)
    yg, cg = _run(m, c0, xs[:N], graph=True)
    st = m.__dict__["_graph_state"]
    assert st["records"] == 2 and st["steps"] == N  # recorded at the start and again after the growth
    for i, (a, b) in enumerate(zip(yg, ye)):
        rel_check(a.float(), b.float(), f"step {i}")
    _same_cache(cg, ce, "cache after growth")
    key_before = st["key"]
    # a weight changed in place: the next step records again and uses it
    print("case weight change", flush=True)
    with torch.no_grad():
        m.o_proj.weight.mul_(1.5)
    ye2, ce2 = _run(m, ce, xs[N:N + 4], graph=False)
    yg2, cg2 = _run(m, cg, xs[N:N + 4], graph=True)
    assert m.__dict__["_graph_state"]["key"] != key_before
    for i, (a, b) in enumerate(zip(yg2, ye2)):
        rel_check(a.float(), b.float(), f"after weight change, step {i}")
    _same_cache(cg2, ce2, "cache after weight change")
    # branching from an older dict leaves the newer one intact
    print("case branch", flush=True)
    saved = cg2["latent"].clone(), cg2["k_rope"].clone()
    yb, cb = _run(m, cg, xs[N + 4:N + 5], graph=True)
    assert torch.equal(cg2["latent"], saved[0]) and torch.equal(cg2["k_rope"], saved[1])
    yr, cr = _run(m, ce, xs[N + 4:N + 5], graph=False)
    rel_check(yb[0].float(), yr[0].float(), "branch step")
    _same_cache(cb, cr, "branched cache")


def test_caches_used_in_turn_fall_back_to_eager():
    m, args = _bf16_module(37)
    B = 2
    ca, cb = _cache(B, 64, args, 38), _cache(B, 80, args, 39)
    g = torch.Generator().manual_seed(40)
    xs = [torch.randn(B, 1, args.d_model, generator=g).to(torch.bfloat16).cuda() for _ in range(8)]
    print("case caches in turn", flush=True)
    ref_a, ref_b = _run(m, ca, xs, graph=False)[0], _run(m, cb, xs, graph=False)[0]
    ya, yb = [], []
    with torch.no_grad():
        for x in xs:  # two caches in turn: every step would record again
            y, ca = m(x, ca, True)
            ya.append(y)
            y, cb = m(x, cb, True)
            yb.append(y)
    assert m.__dict__.get("_graph_off") is True
    assert "_graph_state" not in m.__dict__  # the last recording was released
    for i in range(len(xs)):
        rel_check(ya[i].float(), ref_a[i].float(), f"cache a step {i}")
        rel_check(yb[i].float(), ref_b[i].float(), f"cache b step {i}")


def test_recorded_step_from_an_empty_cache():
    # the first token of a sequence (no cache yet) and the steps after it
    m, args = _bf16_module(41)
    B = 3
    g = torch.Generator().manual_seed(42)
    xs = [torch.randn(B, 1, args.d_model, generator=g).to(torch.bfloat16).cuda() for _ in range(6)]
    print("case empty cache", flush=True)
    ye, ce = _run(m, None, xs, graph=False)
    yg, cg = _run(m, None, xs, graph=True)
    assert m.__dict__["_graph_state"]["records"] == 1
    for i, (a, b) in enumerate(zip(yg, ye)):
        rel_check(a.float(), b.float(), f"step {i}")
    _same_cache(cg, ce, "cache")


def test_recorded_step_at_the_reference_default_dims():
    # params.py defaults: d_model 1792, 14 heads of head_dim 128 (nope 64 + rope 64, v 128),
    # d_latent = q_lora 384, per-head k_rope: the W_UK absorption (K = 64) is outside the few-row
    # kernel's limits, so the recorded step runs hipBLASLt products and the absorb_q kernel
    from types import SimpleNamespace
    from transformer_amd import MLA
    args = SimpleNamespace(d_model=1792, n_heads=14, head_dim=128, d_latent=384, q_lora_rank=384,
                           rope_theta=10000.0, max_seq_len=2048)
    torch.manual_seed(43)
    m = MLA(args)
    g = torch.Generator().manual_seed(43)
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.02)
    m = m.cuda().to(torch.bfloat16)
    assert not m._rows_dims_ok()
    B = 4
    prompt = torch.randn(B, 100, args.d_model, generator=g).to(torch.bfloat16).cuda()
    xs = [torch.randn(B, 1, args.d_model, generator=g).to(torch.bfloat16).cuda() for _ in range(6)]
    print("case reference dims", flush=True)
    with torch.no_grad():
        _, c0 = m(prompt, None, True)
    ye, ce = _run(m, c0, xs, graph=False)
    yg, cg = _run(m, c0, xs, graph=True)
    assert m.__dict__["_graph_state"]["records"] == 1
    for i, (a, b) in enumerate(zip(yg, ye)):
        rel_check(a.float(), b.float(), f"step {i}")
    _same_cache(cg, ce, "cache")


def test_recorded_step_under_inference_mode():
    m, args = _bf16_module(44)
    B = 2
    c0 = _cache(B, 300, args, 45)
    g = torch.Generator().manual_seed(46)
    xs = [torch.randn(B, 1, args.d_model, generator=g).to(torch.bfloat16).cuda() for _ in range(5)]
    print("case inference mode", flush=True)
    ye, ce = _run(m, c0, xs, graph=False)
    yg, c = [], c0
    with torch.inference_mode():
        for x in xs:
            y, c = m(x, c, True)
            yg.append(y)
    assert m.__dict__["_graph_state"]["records"] == 1
    for i, (a, b) in enumerate(zip(yg, ye)):
        rel_check(a.float(), b.float(), f"step {i}")
    _same_cache(c, ce, "cache")


def test_recorded_step_for_fp32_weights_under_bf16_autocast():
    # the reference's generation loop: fp32 model, torch.inference_mode() and bf16 autocast
    # (CLI.py:91,294), with the layer input in fp32 as the reference's RMSNorm leaves it; the
    # module records the step in bf16 from bf16 copies of its weights, bitwise the eager kernels
    m, args = _baseline_module(seed=41)
    assert m.o_proj.weight.dtype == torch.float32
    print("case fp32 weights, bf16 autocast, B=32 L0=1100 N=6", flush=True)
    B, L0, N = 32, 1100, 6
    c0 = _cache(B, L0, args, 42)
    g = torch.Generator().manual_seed(43)
    xs = [torch.randn(B, 1, args.d_model, generator=g).cuda() for _ in range(N)]  # fp32 input

    def run(graph):
        saved = M.AUTO_GRAPH
        M.AUTO_GRAPH = graph
        try:
            ys, c = [], c0
            with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
                for x in xs:
                    y, c = m(x, c, True)
                    ys.append(y)
            return ys, c
        finally:
            M.AUTO_GRAPH = saved

    ye, ce = run(False)
    yg, cg = run(True)
    st = m.__dict__.get("_graph_state")
    assert st is not None and st["graph"] is not None and st["graph"].dtype == torch.bfloat16, "not recorded in bf16"
    for i, (a, b) in enumerate(zip(yg, ye)):
        assert a.dtype == torch.bfloat16 and torch.equal(a, b), f"step {i}"
    _same_cache(cg, ce, "final cache")
    # without autocast the fp32 module computes its projections in fp32 on the eager kernels (no
    # recording: its cache stays fp32, as the reference's)
    m.release_decode_graph()
    with torch.inference_mode():
        y32, c32 = m(xs[0], c0, True)
    assert y32.dtype == torch.float32 and "_graph_state" not in m.__dict__
    assert c32["latent"].dtype == torch.float32 and c32["k_rope"].dtype == torch.float32
    rel_check(y32.float(), ye[0].float(), "fp32 step vs bf16 step")
    # recordings made under inference mode leave torch's RNG usable for recordings outside it
    # (while they live) and for random draws
    z = torch.zeros(8, device="cuda")
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        z.add_(1)
    g2.replay()
    torch.cuda.synchronize()
    assert torch.equal(z, torch.ones(8, device="cuda")) and torch.isfinite(torch.randn(4, device="cuda")).all()
    m.release_decode_graph()


def test_refresh_weights_after_an_update_that_bypasses_the_version_counter():
    # a weight written through .data (as a fused optimizer writing through the storage does) keeps
    # its version counter, so the module's bf16 weight copies and its recorded step stay stale;
    # refresh_weights() rebuilds them, and the step then equals a fresh module's with the new weights
    m, args = _bf16_module(51)
    print("case B=32 L0=1100 refresh", flush=True)
    B, L0 = 32, 1100
    c0 = _cache(B, L0, args, 52)
    g = torch.Generator().manual_seed(53)
    xs = [torch.randn(B, 1, args.d_model, generator=g).to(torch.bfloat16).cuda() for _ in range(3)]
    _run(m, c0, xs[:1], graph=False)  # the eager kernels build the module's bf16 weight copies
    _, c1 = _run(m, c0, xs[:1], graph=True)  # records the step (with copies of its own)
    assert m.__dict__.get("_graph_state") is not None and m.__dict__.get("_derived")
    new_w = {n: (p.float() + 0.01 * torch.randn(p.shape, generator=g).cuda()).to(p.dtype)
             for n, p in m.named_parameters() if n in ("q_down.weight", "kv_down.weight", "k_up.weight")}
    versions = {n: p._version for n, p in m.named_parameters()}
    with torch.no_grad():
        for n, p in m.named_parameters():
            if n in new_w:
                p.data.copy_(new_w[n])
    assert all(p._version == versions[n] for n, p in m.named_parameters()), "the update bumped a version"
    # the next step on the same cache replays the recording, whose weight copies are stale
    stale, _ = _run(m, c1, xs[1:2], graph=True)
    m.refresh_weights()
    assert "_graph_state" not in m.__dict__ and "_derived" not in m.__dict__
    fresh_m, _ = _bf16_module(51)
    fresh_m.load_state_dict(m.state_dict())
    y, c = _run(m, c1, xs[1:2], graph=True)  # c1 again: a branch, copied first
    y_ref, c_ref = _run(fresh_m, c1, xs[1:2], graph=True)
    assert torch.equal(y[0], y_ref[0]), "refreshed module differs from a fresh one"
    _same_cache(c, c_ref, "cache after refresh")
    assert not torch.equal(stale[0], y[0]), "the recording's copies were not stale: the test exercises nothing"
    # the eager kernels' copies are rebuilt too
    ye, _ = _run(m, c1, xs[1:2], graph=False)
    ye_ref, _ = _run(fresh_m, c1, xs[1:2], graph=False)
    assert torch.equal(ye[0], ye_ref[0])
    # the model-level release drops every MLA module's recording
    from transformer_amd import release_decode_graphs
    _run(m, c1, xs[2:3], graph=True)
    model = torch.nn.ModuleList([m, fresh_m])
    assert release_decode_graphs(model) == 2
    assert "_graph_state" not in m.__dict__ and "_graph_state" not in fresh_m.__dict__


def test_fp32_module_without_autocast_keeps_an_fp32_cache():
    # fp32 weights and input, autocast off: the reference's cache is fp32 (torch.cat of the fp32
    # cache and the fp32 projections, transformer.py:215-218, :241-244), so the module records no
    # bf16 step and its eager kernels keep an fp32 cache fp32; attention itself runs in bf16.
    m, args = _baseline_module(seed=44)
    print("case fp32 module B=4 L0=300 N=5", flush=True)
    B, L0, N = 4, 300, 5
    c0 = {k: (v.float() if torch.is_tensor(v) else v) for k, v in _cache(B, L0, args, 45).items()}
    g = torch.Generator().manual_seed(46)
    xs = [torch.randn(B, 1, args.d_model, generator=g).cuda() for _ in range(N)]
    ye, ce = _run(m, c0, xs, graph=False)
    yg, cg = _run(m, c0, xs, graph=True)
    assert "_graph_state" not in m.__dict__, "an fp32 module outside autocast recorded a bf16 step"
    for i, (a, b) in enumerate(zip(yg, ye)):
        assert a.dtype == torch.float32 and torch.equal(a, b), f"fp32 step {i}"
    assert cg["seq_len"] == ce["seq_len"] == L0 + N
    for c in (cg, ce):
        assert c["latent"].dtype == torch.float32 and c["k_rope"].dtype == torch.float32
    assert torch.equal(cg["latent"], ce["latent"]) and torch.equal(cg["k_rope"], ce["k_rope"])
    # the cached rows the caller passed in are carried over unchanged
    assert torch.equal(cg["latent"][:, :L0], c0["latent"]) and torch.equal(cg["k_rope"][:, :, :L0], c0["k_rope"])


_AFTER_AN_INFERENCE_CAPTURE = r'''
import torch
from tests.test_gpu_auto_graph import _bf16_module, _cache, _run, rel_check, _same_cache
with torch.inference_mode():  # a caller's own recording: torch's RNG graph state is made here
    g0 = torch.cuda.CUDAGraph(); y0 = torch.zeros(4, device="cuda")
    with torch.cuda.graph(g0):
        y0.add_(1)
    g0.replay()
m, args = _bf16_module(44)
c0 = _cache(2, 300, args, 45)
g = torch.Generator().manual_seed(46)
xs = [torch.randn(2, 1, args.d_model, generator=g).to(torch.bfloat16).cuda() for _ in range(5)]
ye, ce = _run(m, c0, xs, graph=False)
yg, c = [], c0
with torch.inference_mode():
    for x in xs:
        y, c = m(x, c, True)
        yg.append(y)
assert m.__dict__["_graph_state"]["records"] == 1
for i, (a, b) in enumerate(zip(yg, ye)):
    rel_check(a.float(), b.float(), f"step {i}")
_same_cache(c, ce, "cache")
with torch.inference_mode():  # the caller records again
    g1 = torch.cuda.CUDAGraph(); y1 = torch.zeros(4, device="cuda")
    with torch.cuda.graph(g1):
        y1.add_(1)
    g1.replay()
torch.cuda.synchronize()
assert torch.equal(y1, torch.ones(4, device="cuda")) and torch.isfinite(torch.randn(4, device="cuda")).all()
print("ok")
'''


def test_recorded_step_after_a_recording_made_under_inference_mode():
    # torch's RNG graph state made by a caller's recording under inference mode is held as
    # inference tensors; the module's recording (under inference mode) then begins in the caller's
    # mode, and later recordings still work.  That state lasts for the process, so the case runs
    # in a child process of its own.
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("case recording after an inference-mode capture (child process)", flush=True)
    r = subprocess.run([sys.executable, "-c", _AFTER_AN_INFERENCE_CAPTURE], cwd=root, capture_output=True,
                       text=True, timeout=240)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), (r.returncode, r.stdout[-2000:], r.stderr[-3000:])
