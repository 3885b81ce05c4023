"""Host-side choices that need no GPU: when the decode step's few-row products go to
linear_rows (transformer.py:208-213, :252-254, :300 at T == 1), when a chunk over a cache takes
the absorbed kernel (:249-291 with T > 1), and the backward's workspace falling back to the
recompute path when the stored-dS workspace cannot be allocated."""
from types import SimpleNamespace

import ctypes

import pytest
import torch


def test_rows_path_needs_autograd_off_few_rows_bf16_and_fitting_dims():
    from transformer_amd import MLA, ModelArgs
    m = MLA(ModelArgs.mla_baseline(max_seq_len=64)).to(torch.bfloat16)
    x = torch.zeros(32, 1, m.d_model, dtype=torch.bfloat16)
    assert not m._rows_path(x)  # autograd on: the training path keeps nn.Linear
    with torch.no_grad():
        assert m._rows_path(x)
        assert m._rows_path(torch.zeros(64, 1, m.d_model, dtype=torch.bfloat16))
        assert not m._rows_path(torch.zeros(65, 1, m.d_model, dtype=torch.bfloat16))
        assert not m.float()._rows_path(x.float())  # fp32 arithmetic outside autocast
    # dims the kernel does not take (d_model 64: K not a multiple of 128) stay on nn.Linear
    small = MLA(SimpleNamespace(d_model=64, n_heads=4, head_dim=128, d_latent=64, q_lora_rank=64,
                                max_seq_len=64)).to(torch.bfloat16)
    with torch.no_grad():
        assert not small._rows_path(torch.zeros(1, 1, 64, dtype=torch.bfloat16))


def test_absorbed_chunk_choice():
    # benchmark dims (d_latent 512, nope 128 + rope 64, v 128, shared k_rope): the absorbed kernel
    # costs 1088 multiply-adds per key, head and query against 131072 per key and head to
    # up-project the cache plus 320 per query: short chunks take it, long ones do not
    from transformer_amd import MLA, ModelArgs
    import transformer_amd.mla as M
    m = MLA(ModelArgs.mla_baseline(max_seq_len=64))
    shared = torch.zeros(2, 1, 8, 64)
    with torch.no_grad():
        assert m._absorbed_prefill_ok(2, shared) and m._absorbed_prefill_ok(64, shared)
        assert m._absorbed_prefill_ok(119, shared) and not m._absorbed_prefill_ok(120, shared)
        assert not m._absorbed_prefill_ok(64, torch.zeros(2, 16, 8, 64))  # per-head k_rope
    assert not m._absorbed_prefill_ok(64, shared)  # autograd on: the path with a backward
    saved = M.ABSORBED_PREFILL
    try:
        M.ABSORBED_PREFILL = False
        with torch.no_grad():
            assert not m._absorbed_prefill_ok(64, shared)
    finally:
        M.ABSORBED_PREFILL = saved


def test_rows_fit_limits():
    from transformer_amd import kernels
    assert kernels.rows_fit(128, 4) and kernels.rows_fit(4096, 2624)
    assert not kernels.rows_fit(64, 4) and not kernels.rows_fit(4224, 4) and not kernels.rows_fit(2048, 6)
    assert not kernels.rows_fit(0, 4)


def test_backward_workspace_falls_back_when_the_stored_ds_allocation_fails(monkeypatch):
    from transformer_amd import _lib, kernels
    a = _lib.PrefillBwdArgs()
    a.B, a.H, a.Tq, a.Tk, a.d_nope, a.d_rope, a.d_v, a.causal = 4, 16, 4096, 4096, 128, 64, 128, 1
    full = int(_lib.entry("mla_prefill_bwd_workspace_bytes")(ctypes.byref(a)))
    small = int(_lib.entry("mla_prefill_bwd_workspace_min_bytes")(ctypes.byref(a)))
    assert full > small > 0
    asked = []

    def alloc(nbytes, dev):
        asked.append(nbytes)
        if nbytes > small:
            raise torch.OutOfMemoryError("mocked")
        return torch.empty(max(nbytes, 1), dtype=torch.uint8)

    monkeypatch.setattr(kernels, "_alloc_workspace", alloc)
    ws, nbytes = kernels._bwd_workspace(a, torch.device("cpu"))
    assert asked == [full, small] and nbytes == small and ws.numel() == small
    monkeypatch.setattr(kernels, "BWD_STORED_DS", False)
    asked.clear()
    assert kernels._bwd_workspace(a, torch.device("cpu"))[1] == small and asked == [small]


def test_split_column_product_equals_the_one_product():
    # the down-projection's two-product form, on the host: the same values as x @ W^T, written
    # into the columns of one output
    import transformer_amd.mla as M
    g = torch.Generator().manual_seed(3)
    x = torch.randn(3, 5, 64, generator=g, dtype=torch.float64)
    W = torch.randn(300, 64, generator=g, dtype=torch.float64)
    y = M._linear_split_cols(x, W)
    assert y.shape == (3, 5, 300)
    torch.testing.assert_close(y, x @ W.t(), rtol=1e-12, atol=1e-12)
    assert M._split_pays(24576, 2624) and not M._split_pays(24576, 2560) and not M._split_pays(512, 2624)
    assert not M._split_pays(4096, 200)  # below one 256-column block


def test_eager_ops_take_the_registered_operator_when_it_is_needed():
    # the module layer calls the op bodies directly only when the dispatcher adds nothing: no
    # tracing, dispatch mode, functorch transform, subclass, off-GPU tensor or needed gradient
    from torch._subclasses.fake_tensor import FakeTensorMode
    from transformer_amd import kernels
    need = kernels.dispatcher_needed
    assert not need(()) and not need((1, 2.0, None))
    assert need((torch.zeros(2),))  # a CPU tensor takes the operator (which raises: no CPU path)
    assert need((torch.zeros(2, device="meta"),))  # meta tensors take the fake kernels
    with FakeTensorMode():
        assert need(())
    seen = []
    torch.func.vmap(lambda t: seen.append(need(())) or t)(torch.zeros(3, 2))
    assert seen == [True]
    compiled = torch.compile(lambda t: t + (1 if need(()) else -1), backend="eager", fullgraph=True)
    assert compiled(torch.zeros(1)).item() == 1
    assert all(hasattr(torch.ops.mla_mi355x, n) for n in vars(kernels.eager)) and len(vars(kernels.eager)) == 17
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        kernels.eager.rope(torch.zeros(1, 2, 1, 64, dtype=torch.bfloat16), torch.zeros(4, 32, dtype=torch.bfloat16),
                           torch.zeros(4, 32, dtype=torch.bfloat16), 0, False)


def test_backward_stored_ds_workspace_counts_the_visible_blocks():
    # the stored-dS part of the backward's workspace (its size minus the recompute path's, rounded to
    # 256 bytes) is 2 KiB per 32 x 32 block that the dK/dV pass stores: query block i stores key block j
    # when the block's last query row sees the block's first key (j < ceil(Tk / 32); causal:
    # 32 j <= 32 i + 31 + q_offset), counted here by enumeration; above 8 GiB there is no dS part
    import random
    from transformer_amd import _lib

    def sizes(B, H, Tq, Tk, q_offset, causal):
        a = _lib.PrefillBwdArgs()
        a.B, a.H, a.Tq, a.Tk, a.d_nope, a.d_rope, a.d_v = B, H, Tq, Tk, 128, 64, 128
        a.q_offset, a.causal = q_offset, int(causal)
        full = int(_lib.entry("mla_prefill_bwd_workspace_bytes")(ctypes.byref(a)))
        small = int(_lib.entry("mla_prefill_bwd_workspace_min_bytes")(ctypes.byref(a)))
        return full, small

    def enumerated(B, H, Tq, Tk, q_offset, causal):
        nqb, nkb = (Tq + 31) // 32, (Tk + 31) // 32
        n = sum(1 for i in range(nqb) for j in range(nkb) if not causal or 32 * j <= 32 * i + 31 + q_offset)
        return B * H * n * 2048

    rng = random.Random(5)
    cases = [(1, 1, 32, 32, 0, True), (1, 1, 33, 33, 0, True), (2, 3, 100, 250, 150, True), (1, 2, 64, 31, 0, True),
             (1, 1, 70, 70, 31, True), (1, 1, 70, 70, 32, True), (1, 1, 70, 70, 33, True), (1, 1, 40, 500, 1000, True),
             (3, 2, 77, 45, 0, False), (1, 16, 4096, 4096, 0, True)]
    cases += [(rng.randint(1, 3), rng.randint(1, 4), rng.randint(1, 400), rng.randint(1, 400), rng.choice([0, 0, 1, 31, 32,
              rng.randint(0, 500)]), rng.random() < 0.8) for _ in range(200)]
    for B, H, Tq, Tk, q_offset, causal in cases:
        full, small = sizes(B, H, Tq, Tk, q_offset, causal)
        assert full - ((small + 255) // 256 * 256) == enumerated(B, H, Tq, Tk, q_offset, causal), \
            (B, H, Tq, Tk, q_offset, causal)
    full, small = sizes(16, 16, 16384, 16384, 0, True)  # 17.2 GB of dS blocks: over the cap, recompute path
    assert full == small
