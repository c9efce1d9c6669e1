"""Derived end-to-end bound for the W8A8 attention output (helper of the GPU int8 tests).

The recipe (Project/kernels/k008_int8_gemm.py:189-223) re-quantises the fp16 attention context
per token (``_quant_rows``, :148-151) before the int8 out projection (:221). Our context and the
recipe's context agree to the attention predicate, not bit for bit, so a context value that sits
near a quantisation boundary can round to the neighbouring int8 code. Everything after that
rounding is exact integer arithmetic followed by the fp32 dequantisation, so the output
difference it causes is bounded by the code flips themselves:

    y = fp32(acc) * (s_a * s_w[n]) + b[n],   acc = sum_k q[k] * w_i8[n, k]
    |Y_ours - Y_recipe| <= s_w[n] * ( s_ours * sum_k |q_ours[k] - q_recipe[k]| * |w_i8[n, k]|
                                     + |acc_recipe| * |s_ours - s_recipe| )

for the exact real values Y; the computed fp32 values add at most a few fp32 roundings of each
term (``slack``). ``check`` asserts that every code differs by at most one step, that every
output element meets the bound, and returns the predicate's pass fraction against the recipe.
"""
import numpy as np
import torch

from oracle import int8 as OI
from oracle.predicate import compare_outputs

F32_EPS = 2.0 ** -24


def check(ctx_ours, ctx_recipe, out_w, out_s, out_b, out_ours):
    """ctx_* [T, d] (fp16 values), out_w [N, d] int8, out_s [N], out_b [N], out_ours [T, N] (the
    kernel's output). Returns (pass_fraction, stats dict)."""
    c_o = np.asarray(torch.as_tensor(ctx_ours).float().cpu().numpy(), dtype=np.float32)
    c_r = np.asarray(torch.as_tensor(ctx_recipe).float().cpu().numpy(), dtype=np.float32)
    q_o, s_o = OI.quant_rows(c_o)
    q_r, s_r = OI.quant_rows(c_r)
    dq = np.abs(q_o.astype(np.int32) - q_r.astype(np.int32))
    assert int(dq.max()) <= 1, f"a requantised context code moved by {int(dq.max())} steps"
    acc_o = OI.int8_gemm(q_o, out_w).astype(np.float64)
    acc_r = OI.int8_gemm(q_r, out_w).astype(np.float64)
    y_o = OI.dequant(acc_o.astype(np.int32), s_o, out_s, out_b).astype(np.float64)
    y_r = OI.dequant(acc_r.astype(np.int32), s_r, out_s, out_b).astype(np.float64)
    sw = np.asarray(out_s, np.float64)[None, :]
    so = np.asarray(s_o, np.float64)[:, None]
    sr = np.asarray(s_r, np.float64)[:, None]
    flips = dq.astype(np.float64) @ np.abs(np.asarray(out_w, np.float64)).T   # sum |dq| |w|
    bound = sw * (so * flips + np.abs(acc_r) * np.abs(so - sr))
    slack = 8 * F32_EPS * (np.abs(acc_o) * so * sw + np.abs(acc_r) * sr * sw
                           + np.abs(y_o) + np.abs(y_r))
    diff = np.abs(y_o - y_r)
    worst = float((diff - bound - slack).max())
    assert worst <= 0.0, f"output exceeds the code-flip bound by {worst:.3g}"
    # the kernel's output is the fp32 value of our own codes rounded once to its dtype
    out = torch.as_tensor(out_ours).float().cpu()
    assert torch.equal(out, torch.from_numpy(y_o.astype(np.float32)).to(out_ours.dtype).float())
    r = compare_outputs(torch.from_numpy(y_r.astype(np.float32)), out)
    frac = 1.0 - r.failed_elements / max(1, r.total_elements)
    stats = {"codes_moved": int((dq > 0).sum()), "codes": int(dq.size),
             "rows_with_moved_codes": int((dq.max(axis=1) > 0).sum()), "rows": int(dq.shape[0]),
             "max_diff": float(diff.max()), "max_bound": float(bound.max()),
             "pass_fraction": frac, "predicate": r.summary()}
    return frac, stats
