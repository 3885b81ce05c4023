"""Load the reference golden vectors (tests/golden/mla_ref_golden.npz)."""
import os

import numpy as np
import torch

from oracle.mla_oracle import MLADims

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "mla_ref_golden.npz")


def bf16_from_bits(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.astype(np.uint16).view(np.int16)).view(torch.bfloat16)


class Golden:
    def __init__(self, path=PATH):
        z = np.load(path, allow_pickle=False)
        self.raw = {k: z[k] for k in z.files}
        d = {k[5:]: self.raw[k].item() for k in self.raw if k.startswith("dims.")}
        self.dims = MLADims.reference(d_model=int(d["d_model"]), n_heads=int(d["n_heads"]),
                                      head_dim=int(d["head_dim"]), d_latent=int(d["d_latent"]),
                                      q_lora_rank=int(d["q_lora_rank"]), rope_theta=float(d["rope_theta"]),
                                      max_seq_len=int(d["max_seq_len"]))
        self.weights = {k[2:]: bf16_from_bits(self.raw[k]).float() for k in self.raw if k.startswith("w.")}

    def t(self, key) -> torch.Tensor:
        return torch.from_numpy(np.array(self.raw[key]))


def load_golden():
    return Golden()
