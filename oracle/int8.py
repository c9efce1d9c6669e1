"""numpy restatement of the W8A8 int8 projection recipe — test infrastructure only.

Restates Project/kernels/k008_int8_gemm.py:
  ``_quant_rows``  (:148-151)  per-row activation scale  s = clamp(amax, 1e-6) / 127,
                               q = round_half_even(t / s) -> int8;
  ``_int8_pack``   (:154-158)  per-output-channel weight scale s = clamp(amax / 127, 1e-8);
                               the reference stores W_i8 transposed [K, N]; this restatement
                               returns [N, K] (the library's operand layout) — the integer
                               values are identical;
  ``_int8_linear`` (:181-185)  acc = A_i8 @ W_i8^T (torch._int_mm, exact int32),
                               y = fp32(acc) * (s_a * s_w) + b in fp32, each op rounded.
All arithmetic is float32 (IEEE, no fused multiply-add) exactly as torch performs it, so the
library's outputs are compared bit for bit.

``int8_gemm`` computes the integer product through float64 BLAS, which is exact because every
partial sum is an integer of magnitude <= K * 128 * 128 < 2**53.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


def _to_i8(r: np.ndarray) -> np.ndarray:
    """``.to(torch.int8)`` of the rounded quotients. They lie in [-127, 127] for finite rows;
    a NaN (a row holding NaN has a NaN scale, k008:150, torch's amax and clamp propagate it)
    converts to 0, as the GPU's float-to-integer conversion does."""
    with np.errstate(invalid="ignore"):
        return np.where(np.isnan(r), 0, r).astype(np.int8)


def quant_rows(t: np.ndarray):
    """Activation recipe (k008:148-151): returns (int8 [N, K], fp32 scale [N])."""
    t = np.asarray(t, dtype=F32)
    amax = np.abs(t).max(axis=-1)                  # NaN-propagating, as torch.amax
    s = (np.maximum(amax, F32(1e-6)) / F32(127.0)).astype(F32)   # np.maximum keeps NaN, as clamp
    with np.errstate(invalid="ignore"):
        r = np.rint(t / s[:, None])
    return _to_i8(r), s


def quant_weight(w: np.ndarray):
    """Weight recipe (k008:154-158): returns (int8 [N, K], fp32 scale [N])."""
    w = np.asarray(w, dtype=F32)
    s = np.maximum(np.abs(w).max(axis=1) / F32(127.0), F32(1e-8)).astype(F32)
    with np.errstate(invalid="ignore"):
        r = np.rint(w / s[:, None])
    return _to_i8(r), s


def int8_gemm(a_i8: np.ndarray, w_i8: np.ndarray) -> np.ndarray:
    """Exact int32 accumulators of a_i8 [M, K] @ w_i8 [N, K]^T."""
    a = np.asarray(a_i8)
    w = np.asarray(w_i8)
    K = a.shape[1]
    if K * 128 * 128 >= 2 ** 53:
        raise ValueError("K too large for exact float64 accumulation")
    acc = a.astype(np.float64) @ w.astype(np.float64).T
    return acc.astype(np.int64).astype(np.int32)


def dequant(acc: np.ndarray, s_a: np.ndarray, s_w: np.ndarray, bias=None) -> np.ndarray:
    """y = fp32(acc) * (s_a * s_w) + b, each operation rounded to fp32."""
    y = np.asarray(acc).astype(F32)
    sc = (np.asarray(s_a, F32)[:, None] * np.asarray(s_w, F32)[None, :]).astype(F32)
    y = (y * sc).astype(F32)
    if bias is not None:
        y = (y + np.asarray(bias, F32)[None, :]).astype(F32)
    return y


def int8_linear(h: np.ndarray, w_i8: np.ndarray, s_w: np.ndarray, bias=None):
    """h [N, K] fp32 -> (y fp32 [N, out], acc int32) via per-token quantisation."""
    a8, s_a = quant_rows(h)
    acc = int8_gemm(a8, w_i8)
    return dequant(acc, s_a, s_w, bias), acc


def pack_block(params):
    """Quantised weights of one block: packed QKV [3d, d] and out-proj [d, d] (k008:161-178)."""
    import torch  # local: keep the numpy recipe importable without torch
    w_qkv = torch.cat([params[f"{n}.weight"].float() for n in ("q_proj", "k_proj", "v_proj")]).numpy()
    b_qkv = torch.cat([params[f"{n}.bias"].float() for n in ("q_proj", "k_proj", "v_proj")]).numpy()
    wq, sq = quant_weight(w_qkv)
    wo, so = quant_weight(params["out_proj.weight"].float().numpy())
    return {"qkv_w": wq, "qkv_s": sq, "qkv_b": b_qkv.astype(F32),
            "out_w": wo, "out_s": so, "out_b": params["out_proj.bias"].float().numpy().astype(F32)}


def int8_self_attention(x, params, num_heads: int, causal: bool = False, rows=None):
    """The attention half of ``block_forward`` (k008_int8_gemm.py:189-225) on CPU.

    x [B, S, d] (fp16 values) -> quantised QKV projection -> fp16 qkv (:197) -> fp32-math
    attention with the probabilities rounded to fp16 before P·V (:108, :218) -> context rounded
    to fp16 (the fp16 attention output, :207) -> quantised out
    projection (:221). Returns a dict with the fp16 qkv, the fp16 context and the fp32 output;
    ``rows`` optionally restricts the context/output to a subset of flattened token rows.
    """
    import torch
    from .attention import attention_core

    pk = pack_block(params)
    B, S, d = x.shape
    hd = d // num_heads
    h = x.float().reshape(B * S, d).numpy()
    qkv32, _ = int8_linear(h, pk["qkv_w"], pk["qkv_s"], pk["qkv_b"])
    qkv16 = torch.from_numpy(qkv32.astype(np.float16))
    q5 = qkv16.float().view(B, S, 3, num_heads, hd)
    q, k, v = (q5[:, :, i].transpose(1, 2).contiguous() for i in range(3))
    # fp32 math; probabilities rounded to fp16 before P·V (p.to(tl.float16), k008:108; the
    # eager branch's softmax(...).half(), :218)
    ctx = attention_core(q, k, v, hd ** -0.5, causal, probs_dtype=torch.float16)
    ctx16 = ctx.transpose(1, 2).reshape(B * S, d).to(torch.float16)
    sel = ctx16 if rows is None else ctx16[rows]
    y, _ = int8_linear(sel.float().numpy(), pk["out_w"], pk["out_s"], pk["out_b"])
    return {"qkv16": qkv16, "ctx16": ctx16, "out": torch.from_numpy(y)}


def pack_ffn(params):
    """Quantised FFN weights of one block (``_int8_cache``, k008_int8_gemm.py:174-176):
    ffn_in [ffn, d] and ffn_out [d, ffn] as [N, K] int8 with per-output-channel scales."""
    w1, s1 = quant_weight(params["ffn_in.weight"].float().numpy())
    w2, s2 = quant_weight(params["ffn_out.weight"].float().numpy())
    return {"f1_w": w1, "f1_s": s1, "f1_b": params["ffn_in.bias"].float().numpy().astype(F32),
            "f2_w": w2, "f2_s": s2, "f2_b": params["ffn_out.bias"].float().numpy().astype(F32)}


def int8_transformer_block(x, params, num_heads: int, valid_token_mask=None, causal: bool = False,
                           eps: float = 1e-5):
    """``block_forward`` of k008_int8_gemm.py:189-234 for an fp32 model, on CPU.

    norm1 (fp32, :195) -> int8 QKV -> fp16 qkv (:196-197) -> attention in fp32 math on the fp16
    qkv with the key mask, probabilities rounded to fp16 before P·V (:108, :218), context
    rounded to fp16 (:206-219) -> int8 out projection of the
    context (:221) -> masked rows of it zeroed (:223-224) -> x + attn_out (:225) -> norm2
    (:227) -> int8 ffn_in (:228) -> exact GELU in fp32 (:229) -> int8 ffn_out (:230) ->
    x + out (:231) -> masked rows zeroed (:232-233). ``params`` uses the block's state-dict keys.
    Returns a dict of the stages (torch fp32 tensors; qkv16/ctx16 fp16), ``out`` [B, S, d].
    """
    import torch
    from .attention import attention_core, layer_norm
    from .block import gelu

    B, S, d = x.shape
    T = B * S
    hd = d // num_heads
    att = {k[len("attention."):]: v for k, v in params.items() if k.startswith("attention.")}
    pk = pack_block(att)
    pf = pack_ffn(params)
    xf = x.float().reshape(T, d)
    rows_valid = None if valid_token_mask is None else valid_token_mask.reshape(T, 1)
    h = layer_norm(xf, params["norm1.weight"].float(), params["norm1.bias"].float(), eps)
    qkv32, _ = int8_linear(h.numpy(), pk["qkv_w"], pk["qkv_s"], pk["qkv_b"])
    qkv16 = torch.from_numpy(qkv32.astype(np.float16))
    q5 = qkv16.float().view(B, S, 3, num_heads, hd)
    q, k, v = (q5[:, :, i].transpose(1, 2).contiguous() for i in range(3))
    ctx = attention_core(q, k, v, hd ** -0.5, causal, valid_token_mask,
                         probs_dtype=torch.float16)               # P rounded (:108, :218)
    ctx16 = ctx.transpose(1, 2).reshape(T, d).to(torch.float16)
    attn_out = torch.from_numpy(int8_linear(ctx16.float().numpy(), pk["out_w"], pk["out_s"],
                                            pk["out_b"])[0])
    if rows_valid is not None:
        attn_out = attn_out.masked_fill(~rows_valid, 0)
    x1 = xf + attn_out
    h2 = layer_norm(x1, params["norm2.weight"].float(), params["norm2.bias"].float(), eps)
    hid = gelu(torch.from_numpy(int8_linear(h2.numpy(), pf["f1_w"], pf["f1_s"], pf["f1_b"])[0]))
    out = torch.from_numpy(int8_linear(hid.numpy(), pf["f2_w"], pf["f2_s"], pf["f2_b"])[0])
    y = x1 + out
    if rows_valid is not None:
        y = y.masked_fill(~rows_valid, 0)
    return {"h": h, "qkv16": qkv16, "ctx16": ctx16, "x1": x1, "h2": h2, "g": hid,
            "out": y.view(B, S, d)}
