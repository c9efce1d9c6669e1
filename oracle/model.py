"""Module-level restatement of the benchmark's model classes — test infrastructure only.

Plays the role of the official script module (``otb``) that the reference's plugin contract
passes to ``build(otb, config)`` (Project/harness/candidate_worker.py:275-294), so the plugin
path can be tested without importing the reference. Names, parameter names and forward
signatures follow torch_transformer_benchmark.py:29-200; arithmetic is delegated to
``oracle.attention``.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import attention as _attn


@dataclass(frozen=True)
class TransformerConfig:
    """torch_transformer_benchmark.py:29-56."""
    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int
    causal: bool

    def validate(self) -> None:
        for name in ("batch_size", "seq_len", "d_model", "num_heads", "ffn_dim", "num_layers"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive")
        if self.d_model % self.num_heads:
            raise ValueError("d_model must be divisible by num_heads")


class BaselineSelfAttention(nn.Module):
    """torch_transformer_benchmark.py:59-122 (same attributes and parameter names)."""

    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__()
        if d_model % num_heads:
            raise ValueError("d_model must be divisible by num_heads")
        self.d_model = d_model
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.scale = self.head_dim ** -0.5
        self.q_proj = nn.Linear(d_model, d_model, bias=True)
        self.k_proj = nn.Linear(d_model, d_model, bias=True)
        self.v_proj = nn.Linear(d_model, d_model, bias=True)
        self.out_proj = nn.Linear(d_model, d_model, bias=True)

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None,
                causal: bool = False) -> torch.Tensor:
        params = {k: v.detach() for k, v in self.state_dict().items()}
        out = _attn.self_attention(x, params, self.num_heads, valid_token_mask, causal)
        return out.to(x.dtype)


class BaselineTransformerBlock(nn.Module):
    """Pre-LN block, torch_transformer_benchmark.py:125-145."""

    def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attention = BaselineSelfAttention(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn_in = nn.Linear(d_model, ffn_dim)
        self.ffn_out = nn.Linear(ffn_dim, d_model)

    def forward(self, x, valid_token_mask, causal):
        x = x + self.attention(self.norm1(x), valid_token_mask, causal)
        x = x + self.ffn_out(F.gelu(self.ffn_in(self.norm2(x)), approximate="none"))
        if valid_token_mask is not None:
            x = x.masked_fill(~valid_token_mask[..., None], 0)
        return x


class BaselineTransformer(nn.Module):
    """torch_transformer_benchmark.py:148-172."""

    def __init__(self, config: TransformerConfig) -> None:
        super().__init__()
        self.config = config
        self.layers = nn.ModuleList(
            [BaselineTransformerBlock(config.d_model, config.num_heads, config.ffn_dim)
             for _ in range(config.num_layers)])
        self.final_norm = nn.LayerNorm(config.d_model)

    def forward(self, x, valid_token_mask=None):
        for layer in self.layers:
            x = layer(x, valid_token_mask, self.config.causal)
        x = self.final_norm(x)
        if valid_token_mask is not None:
            x = x.masked_fill(~valid_token_mask[..., None], 0)
        return x


class UserOptimizedTransformer(BaselineTransformer):
    """The replaceable subclass of the official script (torch_transformer_benchmark.py:175-200)."""
