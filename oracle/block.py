"""CPU restatement of the rest of the transformer block and model (test infrastructure only).

``ffn_half`` restates the second residual branch of BaselineTransformerBlock.forward
(torch_transformer_benchmark.py:141-144): norm2 -> ffn_in (nn.Linear(d_model, ffn_dim), :131) ->
exact GELU (``F.gelu(..., approximate="none")``) -> ffn_out (nn.Linear(ffn_dim, d_model), :132)
-> residual add -> masked_fill of invalid rows. ``transformer_block`` composes it with
``attention.attention_half`` (:139), and ``transformer`` runs the layers and the final norm with
its masked_fill (BaselineTransformer.forward, :160-172). Arithmetic is torch-CPU fp32 (fp64 stays
fp64); ``round_to`` applies the rounding points of a model run in that dtype.

``*_bruteforce`` are fp64 restatements with explicit per-element GELU (math.erf) and per-row
LayerNorm loops; they pin the torch restatement (tests/test_oracle_block.py).
"""
from __future__ import annotations

import math
from typing import Dict, Optional

import numpy as np
import torch

from . import attention as _attn


def gelu(x: torch.Tensor) -> torch.Tensor:
    """Exact GELU, ``x * 0.5 * (1 + erf(x / sqrt(2)))`` (F.gelu with approximate="none",
    torch_transformer_benchmark.py:141), in x's floating dtype promoted to at least fp32."""
    x = x.to(torch.promote_types(x.dtype, torch.float32))
    return x * 0.5 * (1.0 + torch.erf(x * (1.0 / math.sqrt(2.0))))


def _linear(x: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor]) -> torch.Tensor:
    return torch.nn.functional.linear(x, w.to(x.dtype), None if b is None else b.to(x.dtype))


def ffn_half(x: torch.Tensor, params: Dict[str, torch.Tensor],
             valid_token_mask: Optional[torch.Tensor] = None, eps: float = 1e-5,
             round_to: Optional[torch.dtype] = None) -> torch.Tensor:
    """``x + ffn_out(gelu(ffn_in(norm2(x))))`` then ``masked_fill(~mask, 0)``
    (torch_transformer_benchmark.py:141-144). ``params`` holds ``norm2.weight``, ``norm2.bias``,
    ``ffn_in.weight``, ``ffn_in.bias``, ``ffn_out.weight``, ``ffn_out.bias``.

    With ``round_to`` the norm output, the ffn_in output, the GELU output, the ffn_out output and
    the residual sum are each rounded to that dtype (every intermediate tensor of a model run in
    it); None keeps every stage in fp32.
    """
    rnd = (lambda t: t.to(round_to).float()) if round_to is not None else (lambda t: t)
    xf = x.to(torch.promote_types(x.dtype, torch.float32))
    h = rnd(_attn.layer_norm(xf, params.get("norm2.weight"), params.get("norm2.bias"), eps))
    f = rnd(_linear(h, params["ffn_in.weight"], params.get("ffn_in.bias")))
    g = rnd(gelu(f))
    o = rnd(_linear(g, params["ffn_out.weight"], params.get("ffn_out.bias")))
    y = rnd(xf + o)
    if valid_token_mask is not None:
        y = y.masked_fill(~valid_token_mask[..., None], 0)
    return y


def _sub(params: Dict[str, torch.Tensor], prefix: str) -> Dict[str, torch.Tensor]:
    n = len(prefix)
    return {k[n:]: v for k, v in params.items() if k.startswith(prefix)}


def transformer_block(x: torch.Tensor, params: Dict[str, torch.Tensor], num_heads: int,
                      valid_token_mask: Optional[torch.Tensor] = None, causal: bool = False,
                      eps: float = 1e-5, round_to: Optional[torch.dtype] = None,
                      attention_round_to: Optional[torch.dtype] = None) -> torch.Tensor:
    """BaselineTransformerBlock.forward (torch_transformer_benchmark.py:134-145): the attention
    half (``attention.attention_half``) then ``ffn_half``. ``params`` uses the block's state-dict
    keys (``norm1.*``, ``attention.*``, ``norm2.*``, ``ffn_in.*``, ``ffn_out.*``).
    ``attention_round_to`` (default ``round_to``) sets the attention half's rounding points."""
    a_rnd = attention_round_to if attention_round_to is not None else round_to
    x1 = _attn.attention_half(x, params.get("norm1.weight"), params.get("norm1.bias"),
                              _sub(params, "attention."), num_heads, valid_token_mask, causal,
                              eps, a_rnd)
    if round_to is not None:
        x1 = x1.to(round_to).float()
    return ffn_half(x1, params, valid_token_mask, eps, round_to)


def transformer(x: torch.Tensor, params: Dict[str, torch.Tensor], num_layers: int, num_heads: int,
                valid_token_mask: Optional[torch.Tensor] = None, causal: bool = False,
                eps: float = 1e-5, round_to: Optional[torch.dtype] = None) -> torch.Tensor:
    """BaselineTransformer.forward (torch_transformer_benchmark.py:160-172): ``num_layers`` blocks
    (``layers.{i}.*`` keys), then ``final_norm`` and the masked_fill of invalid rows."""
    rnd = (lambda t: t.to(round_to).float()) if round_to is not None else (lambda t: t)
    h = x.to(torch.promote_types(x.dtype, torch.float32))
    for i in range(num_layers):
        h = transformer_block(h, _sub(params, f"layers.{i}."), num_heads, valid_token_mask,
                              causal, eps, round_to)
    y = rnd(_attn.layer_norm(h, params.get("final_norm.weight"), params.get("final_norm.bias"), eps))
    if valid_token_mask is not None:
        y = y.masked_fill(~valid_token_mask[..., None], 0)
    return y


# ---------------------------------------------------------------------------------------------
# fp64 brute force (pins the torch restatement)
# ---------------------------------------------------------------------------------------------

def gelu_bruteforce(x) -> np.ndarray:
    """Element-by-element fp64 ``x * Phi(x)`` with ``Phi(x) = (1 + erf(x / sqrt 2)) / 2`` from
    math.erf."""
    x = np.asarray(x, dtype=np.float64)
    flat = x.reshape(-1)
    out = np.empty_like(flat)
    for i, v in enumerate(flat):
        out[i] = v * 0.5 * (1.0 + math.erf(v / math.sqrt(2.0)))
    return out.reshape(x.shape)


def ffn_half_bruteforce(x, params: Dict[str, np.ndarray], valid=None, eps: float = 1e-5) -> np.ndarray:
    """fp64 ``ffn_half``: per-row LayerNorm loops, np.dot linears, per-element math.erf GELU."""
    x = np.asarray(x, dtype=np.float64)
    rows = x.reshape(-1, x.shape[-1])
    h = _attn.layer_norm_bruteforce(rows, params.get("norm2.weight"), params.get("norm2.bias"), eps)
    f = np.dot(h, np.asarray(params["ffn_in.weight"], np.float64).T) + np.asarray(params["ffn_in.bias"], np.float64)
    g = gelu_bruteforce(f)
    o = np.dot(g, np.asarray(params["ffn_out.weight"], np.float64).T) + np.asarray(params["ffn_out.bias"], np.float64)
    y = (rows + o).reshape(x.shape)
    if valid is not None:
        y = np.where(np.asarray(valid)[..., None], y, 0.0)
    return y
