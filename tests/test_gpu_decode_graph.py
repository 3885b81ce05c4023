"""GPU tests of DecodeGraph: the decode step recorded in a HIP graph against the eager
module's cached path (transformer.py:202-300 with T == 1).  The graph is replayed several
times with unrelated eager work and synchronisations between the replays, and every replay
is checked against the eager result."""
import pytest
import torch

from tests.test_gpu_module import _baseline_module, rel_check

pytestmark = pytest.mark.gpu


def _bf16_module(seed):
    m, args = _baseline_module(seed=seed)
    return m.to(torch.bfloat16), args


def test_decode_graph_matches_eager_steps():
    from transformer_amd import DecodeGraph
    m, args = _bf16_module(21)
    g = torch.Generator().manual_seed(22)
    B, T0, N = 2, 100, 6
    prompt = torch.randn(B, T0, args.d_model, generator=g).to(torch.bfloat16).cuda()
    xs = [torch.randn(B, 1, args.d_model, generator=g).to(torch.bfloat16).cuda() for _ in range(N)]
    with torch.no_grad():
        _, c = m(prompt, None, True)
        step = DecodeGraph(m, c, capacity=512)
        ref, ce = [], c
        for x in xs:
            y, ce = m(x, ce, True)
            ref.append(y.clone())
        for i, x in enumerate(xs):
            y = step(x).clone()
            # unrelated eager work and a synchronisation between replays
            junk = torch.randn(256, 256, device="cuda") @ torch.randn(256, 256, device="cuda")
            torch.cuda.synchronize()
            assert torch.isfinite(junk).all()
            rel_check(y.float(), ref[i].float(), f"graph step {i}", rmax=1e-2, rmean=1e-3)
        cg = step.cache()
    assert cg["seq_len"] == ce["seq_len"] == T0 + N
    assert torch.equal(cg["latent"], ce["latent"].to(torch.bfloat16))
    assert torch.equal(cg["k_rope"], ce["k_rope"].to(torch.bfloat16))


def test_decode_graph_input_written_into_its_buffer():
    # a caller that writes its input into step.x (no copy) gets the same steps as one that
    # passes separate tensors
    from transformer_amd import DecodeGraph
    m, args = _bf16_module(23)
    g = torch.Generator().manual_seed(24)
    B, T0 = 2, 70
    prompt = torch.randn(B, T0, args.d_model, generator=g).to(torch.bfloat16).cuda()
    xs = [torch.randn(B, 1, args.d_model, generator=g).to(torch.bfloat16).cuda() for _ in range(3)]
    with torch.no_grad():
        _, c = m(prompt, None, True)
        a, b = DecodeGraph(m, c, capacity=256), DecodeGraph(m, c, capacity=256)
        for x in xs:
            ya = a(x).clone()
            b.x.copy_(x)
            yb = b(b.x).clone()
            assert torch.equal(ya, yb)
    assert torch.equal(a.cache()["latent"], b.cache()["latent"])


def test_decode_graph_capacity_and_shape_checks():
    from transformer_amd import DecodeGraph
    m, args = _bf16_module(23)
    x = torch.randn(1, 8, args.d_model, generator=torch.Generator().manual_seed(24)).to(torch.bfloat16).cuda()
    with torch.no_grad():
        _, c = m(x, None, True)
        with pytest.raises(ValueError):
            DecodeGraph(m, c, capacity=8)  # no room for a token
        step = DecodeGraph(m, c, capacity=9)
        step(x[:, :1])
        with pytest.raises(ValueError):
            step(x[:, :1])  # full
        with pytest.raises(ValueError):
            step(x[:, :2])  # wrong shape


def test_decode_graph_fp32_module_matches_eager():
    # an fp32 module (the reference's default dtype): the projections stay fp32, the cache and
    # the attention are bf16 as in the eager module's cached path
    import transformer_amd.mla as M
    from transformer_amd import DecodeGraph
    m, args = _baseline_module(seed=25)
    saved, M.AUTO_GRAPH = M.AUTO_GRAPH, False  # the reference steps: the eager kernels
    g = torch.Generator().manual_seed(26)
    B, T0, N = 2, 64, 4
    prompt = torch.randn(B, T0, args.d_model, generator=g).cuda()
    xs = [torch.randn(B, 1, args.d_model, generator=g).cuda() for _ in range(N)]
    with torch.no_grad():
        _, c = m(prompt, None, True)
        step = DecodeGraph(m, c, capacity=256)
        ref, ce = [], c
        try:
            for x in xs:
                y, ce = m(x, ce, True)
                ref.append(y.clone())
        finally:
            M.AUTO_GRAPH = saved
        for i, x in enumerate(xs):
            y = step(x).clone()
            assert y.dtype == torch.float32
            rel_check(y, ref[i], f"fp32 graph step {i}", rmax=1e-2, rmean=1e-3)
    assert step.cache()["seq_len"] == T0 + N


def test_decode_graph_owns_the_weights_it_reads():
    # the module's eager path keeps its own concatenated down-projection weight and rebuilds it
    # when asked; a recorded graph must not read that (freed, reused) memory
    from transformer_amd import DecodeGraph
    m, args = _bf16_module(27)
    g = torch.Generator().manual_seed(28)
    B = 2
    prompt = torch.randn(B, 32, args.d_model, generator=g).to(torch.bfloat16).cuda()
    x = torch.randn(B, 1, args.d_model, generator=g).to(torch.bfloat16).cuda()
    with torch.no_grad():
        _, c = m(prompt, None, True)
        y_ref, _ = m(x, c, True)
        step = DecodeGraph(m, c, capacity=64)
        m._down_key = None  # the next eager call rebuilds (and frees) the module's copies
        m.__dict__.pop("_derived", None)
        m(x, c, True)
        junk = [torch.full((4 << 20,), 7.0, dtype=torch.bfloat16, device="cuda") for _ in range(8)]
        y = step(x).clone()
        assert all(bool((j == 7.0).all()) for j in junk)
    rel_check(y.float(), y_ref.float(), "graph after the module's weight copy was rebuilt", rmax=1e-2, rmean=1e-3)
