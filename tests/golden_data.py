"""Loader of the committed golden fixtures (tests/golden/*.npz, written by make_golden.py)."""
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
BLOCK_CASES = ("block_f16_b2s96_d128h2", "block_bf16_b2s80_d128h2", "block_f32_b1s64_d128h2")
TORCH_DTYPE = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def load(name: str) -> dict:
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def params(case: dict, dtype=None) -> dict:
    out = {k.split(":", 1)[1]: torch.from_numpy(np.ascontiguousarray(v)) for k, v in case.items()
           if k.startswith("param:")}
    if dtype is not None:
        out = {k: v.to(dtype) for k, v in out.items()}
    return out
