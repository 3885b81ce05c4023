"""GPU parity of the prefill forward's key split (small grids) and of the edge cases of its key
ranges, against the fp64 oracle's attention (restating SDPA at transformer.py:311-314 and the
masked absorbed prefill at transformer.py:273-291).

When the mirrored q-tile pairs give at most 256 workgroups (B=1 prompts, CLI.py:286,293-296),
mla_prefill_fwd cuts each pair's key tiles into segments whose partials a second kernel merges.
Tolerance: the path's bound, bf16 output within max-abs 2e-2 and mean-abs 2e-3 of the oracle,
LSE within 1e-3; split and unsplit runs of one input agree within 1e-2 (the split keeps its
partials in fp32 and sums in a different order; both round O to bf16).
"""
import ctypes
import math

import pytest
import torch

from tests.gpu_util import check_close, randn_bf16
from tests.test_gpu_prefill import make_inputs, oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import transformer_amd  # noqa: F401
    return torch.ops.mla_mi355x


def _args(d, o, lse, scale, causal, q_offset):
    from transformer_amd import _lib
    from transformer_amd.kernels import _st4
    B, Tq, H, dn = d["q_nope"].shape
    return _lib.PrefillFwdArgs(
        q_nope=d["q_nope"].data_ptr(), q_rope=d["q_rope"].data_ptr(), k_nope=d["k_nope"].data_ptr(),
        k_rope=d["k_rope"].data_ptr(), v=d["v"].data_ptr(), o=o.data_ptr(), lse=lse.data_ptr(),
        B=B, H=H, Tq=Tq, Tk=d["k_nope"].size(1), d_nope=dn, d_rope=64, d_v=128,
        q_nope_stride=_st4(d["q_nope"]), q_rope_stride=_st4(d["q_rope"]), k_nope_stride=_st4(d["k_nope"]),
        k_rope_stride=_st4(d["k_rope"], zero_head=(d["k_rope"].size(2) == 1)), v_stride=_st4(d["v"]),
        o_stride=_st4(o), scale=float(scale), causal=1 if causal else 0, q_offset=int(q_offset),
        workspace=None, workspace_bytes=0)


def run_capi(d, scale, causal, q_offset, split):
    """mla_prefill_fwd through the C ABI, with the key split's workspace (split=True) or without
    one (the unsplit kernel); returns (o, lse, workspace bytes the shape asks for)."""
    from transformer_amd import _lib
    B, Tq, H, _ = d["q_nope"].shape
    o = torch.empty(B, Tq, H, 128, dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(B, H, Tq, dtype=torch.float32, device="cuda")
    a = _args(d, o, lse, scale, causal, q_offset)
    nbytes = int(_lib.entry("mla_prefill_fwd_workspace_bytes")(ctypes.byref(a)))
    ws = None
    if split and nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    torch.cuda.synchronize()
    _lib.check(_lib.entry("mla_prefill_fwd")(ctypes.byref(a), torch.cuda.current_stream().cuda_stream), "fwd")
    torch.cuda.synchronize()
    return o.cpu(), lse.cpu(), nbytes


SPLIT_CASES = [
    # B, Tq, Tk, H, Hr, dn, causal, q_offset
    (1, 1024, 1024, 2, 1, 128, True, 0),     # 4 pairs of 8 q-tiles: 4 segments per pair (8 WGs → S=8 capped by N/8 = 4)
    (2, 700, 700, 3, 3, 64, True, 0),        # per-head k_rope, d_nope 64, Tq % 128 and Tk % 32 != 0
    (1, 100, 3000, 4, 1, 128, False, 0),     # one q-tile over a long key range, 8 segments
    (1, 280, 1280, 2, 1, 128, True, 1000),   # chunk over a cache: q_offset % 32 != 0, Tk % 32 == 0
    (1, 300, 1333, 2, 1, 128, True, 1033),   # q_offset and Tk both off the 32-key grid
    (3, 640, 640, 5, 1, 128, True, 0),
]


@pytest.mark.parametrize("B,Tq,Tk,H,Hr,dn,causal,q_offset", SPLIT_CASES)
def test_split_matches_oracle_and_unsplit(B, Tq, Tk, H, Hr, dn, causal, q_offset):
    print(f"case B={B} Tq={Tq} Tk={Tk} H={H} Hr={Hr} dn={dn} causal={causal} q_offset={q_offset}", flush=True)
    inp = make_inputs(B, Tq, Tk, H, Hr, dn, seed=Tq * 7 + Tk + H)
    scale = 1 / math.sqrt(dn + 64)
    d = {k: v.cuda() for k, v in inp.items()}
    o_s, lse_s, nbytes = run_capi(d, scale, causal, q_offset, split=True)
    assert nbytes > 0, "this shape is meant to take the key split"
    o_u, lse_u, _ = run_capi(d, scale, causal, q_offset, split=False)
    ref_o, ref_lse = oracle(inp, scale, causal, q_offset)
    m_s = check_close(o_s.double(), ref_o, "O (split)")
    m_u = check_close(o_u.double(), ref_o, "O (unsplit)")
    print(f"  split max {m_s['max']:.2e} mean {m_s['mean']:.2e}; unsplit max {m_u['max']:.2e} mean {m_u['mean']:.2e}")
    torch.testing.assert_close(lse_s.double(), ref_lse, rtol=0, atol=1e-3)
    torch.testing.assert_close(lse_u.double(), ref_lse, rtol=0, atol=1e-3)
    assert (o_s.float() - o_u.float()).abs().max().item() <= 1e-2


def test_split_reference_prompt_shape_sampled_heads(ops):
    # the reference's inference prefill: one 2048-token prompt, 16 heads (CLI.py:286,293-296)
    B, T, H = 1, 2048, 16
    inp = make_inputs(B, T, T, H, 1, 128, seed=2048)
    scale = 1 / math.sqrt(192)
    d = {k: v.cuda() for k, v in inp.items()}
    o, lse = ops.prefill_fwd(d["q_nope"], d["q_rope"], d["k_nope"], d["k_rope"], d["v"], scale, True, 0)
    o, lse = o.cpu(), lse.cpu()
    pairs = [(0, 0), (0, 9), (0, 15)]
    ref = oracle(inp, scale, True, 0, heads=pairs)
    for (b, h), (ro, rl) in ref.items():
        m = check_close(o[b, :, h].double(), ro, f"O[b={b},h={h}]")
        print(f"  head {h}: max {m['max']:.2e} mean {m['mean']:.2e} p99 {m.get('p99', float('nan')):.2e}")
        torch.testing.assert_close(lse[b, h].double(), rl, rtol=0, atol=1e-3)


def test_split_is_deterministic(ops):
    inp = {k: v.cuda() for k, v in make_inputs(1, 1024, 1024, 4, 1, 128, seed=29).items()}
    a = ops.prefill_fwd(inp["q_nope"], inp["q_rope"], inp["k_nope"], inp["k_rope"], inp["v"], 0.07, True, 0)
    b = ops.prefill_fwd(inp["q_nope"], inp["q_rope"], inp["k_nope"], inp["k_rope"], inp["v"], 0.07, True, 0)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_split_score_jump_takes_the_rescaling_path():
    # A key in the middle of a long segment outscores the segment's first tile by ~200 (log2) for
    # some rows: the segment's fixed reference max would overflow, so its workgroup votes and
    # recomputes the segment with the rescaling loop; the merge then sees ordinary partials.
    inp = make_inputs(1, 1024, 1024, 2, 1, 128, seed=31)
    q = torch.cat([inp["q_nope"], inp["q_rope"]], -1).float()
    k_jump = (8.0 * q[0, 1000, 0]).to(torch.bfloat16)
    inp["k_nope"][0, 700, 0] = k_jump[:128]
    inp["k_rope"][0, 700, 0] = k_jump[128:]
    scale = 1 / math.sqrt(192)
    d = {k: v.cuda() for k, v in inp.items()}
    o, lse, nbytes = run_capi(d, scale, True, 0, split=True)
    assert nbytes > 0
    ref_o, ref_lse = oracle(inp, scale, True, 0)
    assert torch.isfinite(o.float()).all() and torch.isfinite(lse).all()
    check_close(o.double(), ref_o, "O (split, score jump)")
    torch.testing.assert_close(lse.double(), ref_lse, rtol=0, atol=1e-3)
    qk = (q[0, 700:, 0] @ k_jump.float()) * scale * 1.4426950408889634
    assert qk.max().item() > 130


def _poison_lds(ops):
    """Runs the forward over NaN inputs on a grid that covers every CU, so the LDS of every CU is
    left holding NaN K/V tiles for the next kernel."""
    g = torch.Generator().manual_seed(3)
    B, T, H = 4, 1024, 16
    nan = lambda *s: torch.full(s, float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.prefill_fwd(nan(B, T, H, 128), nan(B, T, H, 64), nan(B, T, H, 128), nan(B, T, 1, 64), nan(B, T, H, 128),
                    0.07, True, 0)
    torch.cuda.synchronize()


def test_q_offset_off_the_key_grid_after_nan_in_lds(ops):
    # A 280-token chunk over a 1000-token cache (Tk = 1280, a multiple of 32; q_offset = 1000 is
    # not): the causal end of each q-tile falls inside a 32-key tile, whose rows past it meet
    # p = 0 in the P V product.  Run unsplit right after a kernel that leaves NaN in LDS.
    inp = make_inputs(1, 280, 1280, 2, 1, 128, seed=37)
    scale = 1 / math.sqrt(192)
    d = {k: v.cuda() for k, v in inp.items()}
    _poison_lds(ops)
    o, lse, _ = run_capi(d, scale, True, 1000, split=False)
    ref_o, ref_lse = oracle(inp, scale, True, 1000)
    check_close(o.double(), ref_o, "O (q_offset 1000, after NaN in LDS)")
    torch.testing.assert_close(lse.double(), ref_lse, rtol=0, atol=1e-3)


def test_per_tile_descriptors_for_key_ranges_past_2_gib(ops):
    # k_nope rows 4 MiB apart: its key range spans more than 2^31 bytes, so the kernel builds a
    # descriptor per tile (ending at the q-tile's last visible key) instead of one per (b, h).
    # q_offset % 32 != 0 puts that end inside a tile; run after NaN in LDS.
    Tq, Tk, H, off = 280, 512, 1, 200
    inp = make_inputs(1, Tq, Tk, H, 1, 128, seed=41)
    st = (1 << 21) + 8192  # elements between key rows: (Tk - 1) * st * 2 bytes > 2^31
    assert (Tk - 1) * st * 2 + 256 >= (1 << 31)
    base = torch.empty(Tk * st, dtype=torch.bfloat16, device="cuda")
    kn = base.as_strided((1, Tk, H, 128), (Tk * st, st, 128, 1))
    kn.copy_(inp["k_nope"].cuda())
    d = {k: v.cuda() for k, v in inp.items()}
    d["k_nope"] = kn
    scale = 1 / math.sqrt(192)
    _poison_lds(ops)
    o, lse, nbytes = run_capi(d, scale, True, off, split=True)
    ref_o, ref_lse = oracle(inp, scale, True, off)
    check_close(o.double(), ref_o, "O (per-tile descriptors)")
    torch.testing.assert_close(lse.double(), ref_lse, rtol=0, atol=1e-3)
    del base
