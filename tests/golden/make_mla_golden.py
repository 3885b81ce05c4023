"""Write golden vectors of the reference MLA module (run once, in the survey container).

The reference (manningwu07/transformer, pure Python/PyTorch) is imported from
``/root/reference`` ONLY by this script, only in the build container, to record
inputs and outputs of ``MLA.forward`` (transformer.py:202-316) and
``RotaryEmbedding`` (transformer.py:29-53).  Nothing from the reference is stored
but numbers: seeded inputs, bf16-rounded weights and the module's outputs.

What the vectors pin that no closed form does: the composition conventions of the
module -- ``qk_rope`` output order (q first, :210), head view layout (:221-222),
rope-last concat (:311-312), cache-dict contents (:295-299), the absorbed branch's
bottom-right mask for chunked prefill (:273-281), and the bf16 RoPE tables (:35-44).

Usage:  python tests/golden/make_mla_golden.py  [--ref /root/reference]
Output: tests/golden/mla_ref_golden.npz
"""
import argparse
import os
import sys
from types import SimpleNamespace

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

# reference dims, scaled down: head_dim 128 => content 64 + rope 64, v 128, per-head k_rope
DIMS = dict(d_model=64, n_heads=4, head_dim=128, d_latent=64, q_lora_rank=64,
            rope_theta=10000.0, max_seq_len=64)
TABLE_ROWS = 16384  # long-context table (config 3 needs >= 16384 rows)
SEED = 1234


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--out", default=os.path.join(HERE, "mla_ref_golden.npz"))
    args = ap.parse_args()
    sys.path.insert(0, args.ref)
    import transformer as ref  # noqa: E402  (reference module, build container only)

    torch.manual_seed(0)
    cfg = SimpleNamespace(**DIMS)
    mla = ref.MLA(cfg).float().eval()

    g = torch.Generator().manual_seed(SEED)
    sd = {}
    for name, p in mla.named_parameters():
        w = (torch.randn(p.shape, generator=g) * 0.02).to(torch.bfloat16).float()
        with torch.no_grad():
            p.copy_(w)
        sd[name] = w
    out = {f"w.{k}": bf16_bits(v) for k, v in sd.items()}
    for k, v in DIMS.items():
        out[f"dims.{k}"] = np.asarray(v)

    # 1) training / no-cache branch (SDPA, :306-316) + backward
    x = torch.randn(2, 24, DIMS["d_model"], generator=g)
    dy = torch.randn(2, 24, DIMS["d_model"], generator=g)
    xr = x.clone().requires_grad_(True)
    y, cache = mla(xr, None, False)
    assert cache is None
    y.backward(dy)
    out.update({"train.x": x.numpy(), "train.dy": dy.numpy(), "train.y": y.detach().numpy(),
                "train.dx": xr.grad.numpy(),
                "train.dk_up": mla.k_up.weight.grad.numpy()})

    with torch.no_grad():
        # 2) absorbed prefill with cache (:249-300, T > 1, no cache yet)
        xp = torch.randn(2, 20, DIMS["d_model"], generator=g)
        yp, c = mla(xp, None, True)
        out.update({"prefill.x": xp.numpy(), "prefill.y": yp.numpy(),
                    "prefill.latent": c["latent"].numpy(), "prefill.k_rope": c["k_rope"].numpy(),
                    "prefill.seq_len": np.asarray(c["seq_len"])})
        # 3) three single-token decode steps (:249-300, T == 1)
        for i in range(3):
            xd = torch.randn(2, 1, DIMS["d_model"], generator=g)
            yd, c = mla(xd, c, True)
            out[f"decode{i}.x"] = xd.numpy()
            out[f"decode{i}.y"] = yd.numpy()
        # 4) chunked prefill on top of the cache (T > 1 with pos_offset, mask :273-281)
        xc = torch.randn(2, 5, DIMS["d_model"], generator=g)
        yc, c = mla(xc, c, True)
        out.update({"chunk.x": xc.numpy(), "chunk.y": yc.numpy(),
                    "chunk.latent": c["latent"].numpy(), "chunk.k_rope": c["k_rope"].numpy(),
                    "chunk.seq_len": np.asarray(c["seq_len"])})

        # 5) RoPE tables of the reference RotaryEmbedding at 16384 rows (sampled rows)
        rot = ref.RotaryEmbedding(64, max_seq_len=TABLE_ROWS, theta=10000.0)
        rows = np.unique(np.concatenate([np.arange(64), np.random.RandomState(SEED).randint(0, TABLE_ROWS, 192),
                                         [TABLE_ROWS - 1]])).astype(np.int64)
        out["rope.rows"] = rows
        out["rope.cos"] = bf16_bits(rot.cos_cached[torch.from_numpy(rows)])
        out["rope.sin"] = bf16_bits(rot.sin_cached[torch.from_numpy(rows)])
        # apply_rope on a fixed input at positions 0..63 (:55-60)
        xr_ = torch.randn(3, 64, 64, generator=g)
        out["rope.x"] = xr_.numpy()
        cos = rot.cos_cached[:64].float()
        sin = rot.sin_cached[:64].float()
        out["rope.y"] = ref.apply_rope(xr_, cos, sin).numpy()

    np.savez_compressed(args.out, **out)
    print("wrote", args.out, sum(v.nbytes for v in out.values()), "bytes")


if __name__ == "__main__":
    main()
