"""Dense CPU restatement of the reference attention block (test infrastructure only).

``self_attention`` restates ``BaselineSelfAttention.forward``
(torch_transformer_benchmark.py:85-122) op for op in torch-CPU fp32:
q/k/v projections (:93-95) -> head split (:77-83) -> scores * scale (:97) -> causal mask
(:99-103) -> key mask (:105-108) -> fp32 softmax (:110-111) -> P·V (:112) -> head merge
(:113-117) -> out_proj (:118) -> output-row mask (:120-121).

``*_bruteforce`` are independent fp64 numpy restatements with explicit per-row loops; they pin
the torch restatement (tests/test_oracle.py).
"""
from __future__ import annotations

from typing import Dict, Optional

import numpy as np
import torch

PARAM_NAMES = ("q_proj", "k_proj", "v_proj", "out_proj")


def split_heads(t: torch.Tensor, num_heads: int) -> torch.Tensor:
    """[B, S, d] -> [B, H, S, hd] (torch_transformer_benchmark.py:77-83)."""
    B, S, d = t.shape
    return t.view(B, S, num_heads, d // num_heads).transpose(1, 2).contiguous()


def merge_heads(t: torch.Tensor) -> torch.Tensor:
    """[B, H, S, hd] -> [B, S, d] (torch_transformer_benchmark.py:113-117)."""
    B, H, S, hd = t.shape
    return t.transpose(1, 2).contiguous().view(B, S, H * hd)


def attention_core(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                   causal: bool = False, valid_token_mask: Optional[torch.Tensor] = None,
                   probs_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Scores -> masks -> fp32 softmax -> P·V on [B, H, S, hd] (torch_transformer_benchmark.py:97-112).

    ``probs_dtype`` reproduces the ``.to(dtype=x.dtype)`` rounding of the probabilities (:111)
    when the block runs in a 16-bit dtype; None keeps them fp32.
    """
    S_q, S_k = q.shape[-2], k.shape[-2]
    scores = torch.matmul(q, k.transpose(-2, -1)) * scale
    if causal:
        causal_mask = torch.ones((S_q, S_k), dtype=torch.bool).triu(diagonal=1)
        scores = scores.masked_fill(causal_mask, float("-inf"))
    if valid_token_mask is not None:
        scores = scores.masked_fill(~valid_token_mask[:, None, None, :], float("-inf"))
    # fp32 softmax (:111); an fp64 caller keeps fp64 (used for error-bound references)
    probs = torch.softmax(scores.to(torch.promote_types(scores.dtype, torch.float32)), dim=-1)
    if probs_dtype is not None:
        probs = probs.to(probs_dtype).to(v.dtype)
    return torch.matmul(probs.to(v.dtype), v)


def self_attention(x: torch.Tensor, params: Dict[str, torch.Tensor], num_heads: int,
                   valid_token_mask: Optional[torch.Tensor] = None, causal: bool = False,
                   probs_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """fp32 CPU forward of the block; ``params`` maps ``'<proj>.weight'/'<proj>.bias'``.

    All arithmetic is fp32 on whatever values are passed (callers pass the 16-bit-rounded
    inputs and weights upcast to fp32 for the fp16/bf16 configurations).
    """
    x = x.float()
    p = {n: t.float() for n, t in params.items()}
    d = x.shape[-1]
    scale = (d // num_heads) ** -0.5
    q = split_heads(torch.nn.functional.linear(x, p["q_proj.weight"], p["q_proj.bias"]), num_heads)
    k = split_heads(torch.nn.functional.linear(x, p["k_proj.weight"], p["k_proj.bias"]), num_heads)
    v = split_heads(torch.nn.functional.linear(x, p["v_proj.weight"], p["v_proj.bias"]), num_heads)
    ctx = merge_heads(attention_core(q, k, v, scale, causal, valid_token_mask, probs_dtype))
    out = torch.nn.functional.linear(ctx, p["out_proj.weight"], p["out_proj.bias"])
    if valid_token_mask is not None:
        out = out.masked_fill(~valid_token_mask[..., None], 0)
    return out


def qkv_projection(x: torch.Tensor, params: Dict[str, torch.Tensor]) -> torch.Tensor:
    """Packed projection ``[B, S, 3d]`` = x·[Wq;Wk;Wv]^T + [bq;bk;bv] in fp32
    (the packing of Project/submission/dispatcher_region.py:789-792)."""
    w = torch.cat([params[f"{n}.weight"].float() for n in PARAM_NAMES[:3]], dim=0)
    b = torch.cat([params[f"{n}.bias"].float() for n in PARAM_NAMES[:3]], dim=0)
    return torch.nn.functional.linear(x.float(), w, b)


def layer_norm(x: torch.Tensor, weight: Optional[torch.Tensor], bias: Optional[torch.Tensor],
               eps: float = 1e-5) -> torch.Tensor:
    """nn.LayerNorm over the last dimension (``norm1`` of torch_transformer_benchmark.py:128,
    applied at :139) in torch-CPU fp32 (fp64 stays fp64): biased variance, eps inside the
    square root, then the elementwise affine map."""
    x = x.to(torch.promote_types(x.dtype, torch.float32))
    mean = x.mean(-1, keepdim=True)
    var = ((x - mean) ** 2).mean(-1, keepdim=True)
    y = (x - mean) / torch.sqrt(var + eps)
    if weight is not None:
        y = y * weight.to(y.dtype)
    if bias is not None:
        y = y + bias.to(y.dtype)
    return y


def attention_half(x: torch.Tensor, norm_weight: Optional[torch.Tensor],
                   norm_bias: Optional[torch.Tensor], params: Dict[str, torch.Tensor],
                   num_heads: int, valid_token_mask: Optional[torch.Tensor] = None,
                   causal: bool = False, eps: float = 1e-5,
                   round_to: Optional[torch.dtype] = None) -> torch.Tensor:
    """``x + attention(norm1(x), valid_token_mask, causal)``, the first residual branch of
    BaselineTransformerBlock.forward (torch_transformer_benchmark.py:139), in fp32.

    ``round_to`` applies the roundings of a block run in that dtype: the norm output, the
    attention output (:118-122, ``.to(x.dtype)`` of the module) and the residual sum are each
    rounded to it; None keeps every stage fp32.
    """
    rnd = (lambda t: t.to(round_to).float()) if round_to is not None else (lambda t: t)
    xf = x.float()
    h = rnd(layer_norm(xf, norm_weight, norm_bias, eps))
    a = rnd(self_attention(h, params, num_heads, valid_token_mask, causal))
    return rnd(xf + a)


# ---------------------------------------------------------------------------------------------
# fp64 brute force (pins the torch restatement)
# ---------------------------------------------------------------------------------------------

def layer_norm_bruteforce(x, weight=None, bias=None, eps: float = 1e-5) -> np.ndarray:
    """Per-row fp64 LayerNorm with explicit loops over the row."""
    x = np.asarray(x, dtype=np.float64)
    rows = x.reshape(-1, x.shape[-1])
    K = rows.shape[1]
    w = np.ones(K) if weight is None else np.asarray(weight, dtype=np.float64)
    b = np.zeros(K) if bias is None else np.asarray(bias, dtype=np.float64)
    out = np.empty_like(rows)
    for r in range(rows.shape[0]):
        mean = 0.0
        for j in range(K):
            mean += rows[r, j]
        mean /= K
        var = 0.0
        for j in range(K):
            var += (rows[r, j] - mean) ** 2
        var /= K
        inv = 1.0 / np.sqrt(var + eps)
        for j in range(K):
            out[r, j] = (rows[r, j] - mean) * inv * w[j] + b[j]
    return out.reshape(x.shape)


def attention_core_bruteforce(q, k, v, scale: float, causal: bool = False, valid=None) -> np.ndarray:
    """Per-query-row fp64 softmax attention on [B, H, S, hd] arrays."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, H, S_q, hd = q.shape
    S_k = k.shape[2]
    out = np.empty((B, H, S_q, v.shape[3]), dtype=np.float64)
    for b in range(B):
        for h in range(H):
            for i in range(S_q):
                s = np.array([float(np.dot(q[b, h, i], k[b, h, j])) * scale for j in range(S_k)])
                allowed = np.ones(S_k, dtype=bool)
                if causal:
                    allowed &= np.arange(S_k) <= i
                if valid is not None:
                    allowed &= np.asarray(valid[b], dtype=bool)
                if not allowed.any():
                    out[b, h, i] = np.nan
                    continue
                s = np.where(allowed, s, -np.inf)
                e = np.exp(s - s[allowed].max())
                pr = e / e.sum()
                out[b, h, i] = pr @ v[b, h]
    return out


def self_attention_bruteforce(x, params: Dict[str, np.ndarray], num_heads: int, causal: bool = False,
                              valid=None) -> np.ndarray:
    """fp64 numpy forward of the whole block with per-row attention loops."""
    x = np.asarray(x, dtype=np.float64)
    p = {n: np.asarray(t, dtype=np.float64) for n, t in params.items()}
    B, S, d = x.shape
    hd = d // num_heads

    def lin(t, name):
        return t @ p[f"{name}.weight"].T + p[f"{name}.bias"]

    def heads(t):
        return t.reshape(B, S, num_heads, hd).transpose(0, 2, 1, 3)

    q, k, v = heads(lin(x, "q_proj")), heads(lin(x, "k_proj")), heads(lin(x, "v_proj"))
    ctx = attention_core_bruteforce(q, k, v, hd ** -0.5, causal, valid)
    ctx = ctx.transpose(0, 2, 1, 3).reshape(B, S, d)
    out = lin(ctx, "out_proj")
    if valid is not None:
        out = np.where(np.asarray(valid, dtype=bool)[..., None], out, 0.0)
    return out
