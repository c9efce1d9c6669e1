"""Writes the committed golden fixtures of this directory from the CPU oracle.

Run from the repository root:  python tests/golden/make_golden.py

Inputs are drawn with numpy's PCG64 generator (seeded, machine independent) and rounded to the
case's dtype; bf16 values are stored as the fp32 numbers they equal exactly. Expected outputs
come from the oracle (fp32 math on the rounded inputs; the numpy int8 recipe), so the GPU tests
can compare the HIP path against fixed data without running the oracle, and the CPU tests
check that the oracle still reproduces them. The reference ships no tensor fixtures of its own
for this path; these are the oracle's, pinned by tests/test_oracle.py.
Files are plain ``.npz`` (no pickled objects).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import attention as OA  # noqa: E402
from oracle import int8 as OI  # noqa: E402

PROJ = ("q_proj", "k_proj", "v_proj", "out_proj")


def _round(a: np.ndarray, dtype: str) -> np.ndarray:
    t = torch.from_numpy(a.astype(np.float32))
    if dtype == "f16":
        return t.to(torch.float16).numpy()
    if dtype == "bf16":
        return t.to(torch.bfloat16).float().numpy()
    return t.numpy()


def _params(rng, d: int, dtype: str, std: float):
    out = {}
    for n in PROJ:
        out[f"{n}.weight"] = _round(rng.standard_normal((d, d)) * std, dtype)
        out[f"{n}.bias"] = _round(rng.uniform(-d ** -0.5, d ** -0.5, d), dtype)
    return out


def _lengths_mask(B: int, S: int, lengths) -> np.ndarray:
    return np.arange(S)[None, :] < np.asarray(lengths)[:, None]


def block_case(name: str, B: int, S: int, d: int, H: int, dtype: str, seed: int, lengths):
    rng = np.random.Generator(np.random.PCG64(seed))
    params = _params(rng, d, dtype, d ** -0.5)
    x = _round(rng.standard_normal((B, S, d)), dtype)
    mask = _lengths_mask(B, S, lengths)
    x = np.where(mask[..., None], x, 0).astype(x.dtype)
    pt = {k: torch.from_numpy(v.astype(np.float32)) for k, v in params.items()}
    xt = torch.from_numpy(x.astype(np.float32))
    mt = torch.from_numpy(mask)
    out = {"x": x, "mask": mask, "heads": np.int64(H), "dtype": np.array(dtype)}
    out.update({f"param:{k}": v for k, v in params.items()})
    with torch.no_grad():
        out["out_noncausal"] = OA.self_attention(xt, pt, H, mt, causal=False).numpy()
        out["out_causal"] = OA.self_attention(xt, pt, H, mt, causal=True).numpy()
    np.savez(os.path.join(HERE, name + ".npz"), **out)


def attention_case(name: str, B: int, S: int, H: int, hd: int, seed: int, lengths):
    """Raw kernel case: q, k, v [B, S, H, hd] fp16 with a key mask."""
    rng = np.random.Generator(np.random.PCG64(seed))
    q, k, v = (_round(rng.standard_normal((B, S, H, hd)) * s, "f16") for s in (1.0, 1.0, 1.0))
    mask = _lengths_mask(B, S, lengths)
    tq, tk, tv = (torch.from_numpy(a.astype(np.float32)).transpose(1, 2) for a in (q, k, v))
    res = {"q": q, "k": k, "v": v, "mask": mask}
    with torch.no_grad():
        for causal in (False, True):
            o = OA.attention_core(tq, tk, tv, hd ** -0.5, causal, torch.from_numpy(mask))
            res["ctx_causal" if causal else "ctx_noncausal"] = o.transpose(1, 2).numpy()
    np.savez(os.path.join(HERE, name + ".npz"), **res)


def int8_case(name: str, B: int, S: int, d: int, H: int, seed: int):
    rng = np.random.Generator(np.random.PCG64(seed))
    params = {k: v.astype(np.float32) for k, v in _params(rng, d, "f32", 0.02).items()}
    x = _round(rng.standard_normal((B, S, d)), "f16")
    pt = {k: torch.from_numpy(v) for k, v in params.items()}
    want = OI.int8_self_attention(torch.from_numpy(x), pt, H, False)
    pk = OI.pack_block(pt)
    xq, sx = OI.quant_rows(x.astype(np.float32).reshape(B * S, d))
    acc = OI.int8_gemm(xq, pk["qkv_w"])
    res = {"x": x, "heads": np.int64(H), "x_i8": xq, "x_scale": sx, "qkv_acc": acc,
           "qkv16": want["qkv16"].numpy(), "ctx16": want["ctx16"].numpy(),
           "out_recipe": want["out"].numpy()}
    res.update({f"param:{k}": v for k, v in params.items()})
    np.savez(os.path.join(HERE, name + ".npz"), **res)


def quant_case(name: str):
    """Rows that exercise the recipe's edge cases: zeros, exact ties, the row maximum, tiny rows."""
    K = 32
    rows = [np.zeros(K), np.full(K, 3.0), np.linspace(-1.0, 1.0, K), np.full(K, 1e-9)]
    tie = np.zeros(K)
    tie[0] = 127.0
    tie[1:6] = [0.5, 1.5, 2.5, -0.5, -2.5]     # exact .5 multiples of the scale 1.0
    rows.append(tie)
    rng = np.random.Generator(np.random.PCG64(7))
    rows += list(rng.standard_normal((11, K)) * rng.uniform(1e-3, 1e3, (11, 1)))
    # non-finite rows: torch's amax/clamp propagate NaN into the scale (every code 0); an inf
    # element makes the scale inf (its own code NaN -> 0, the finite ones round to 0)
    nan_row = rng.standard_normal(K)
    nan_row[3] = np.nan
    inf_row = rng.standard_normal(K)
    inf_row[5] = -np.inf
    rows += [nan_row, inf_row]
    x = np.stack(rows).astype(np.float32)
    q0, s0 = OI.quant_rows(x)
    q1, s1 = OI.quant_weight(x)
    np.savez(os.path.join(HERE, name + ".npz"), x=x, q_act=q0, s_act=s0, q_w=q1, s_w=s1)


def main():
    block_case("block_f16_b2s96_d128h2", 2, 96, 128, 2, "f16", 11, [96, 70])
    block_case("block_bf16_b2s80_d128h2", 2, 80, 128, 2, "bf16", 12, [80, 41])
    block_case("block_f32_b1s64_d128h2", 1, 64, 128, 2, "f32", 13, [64])
    attention_case("attn_f16_hd128_b1s80h2", 1, 80, 2, 128, 14, [67])
    int8_case("int8_block_b1s64_d128h2", 1, 64, 128, 2, 15)
    quant_case("quant_rows_cases")
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
