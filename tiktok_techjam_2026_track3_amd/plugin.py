"""The reference's three insertion points for an optimised attention block.

1. module swap   — ``swap_attention(model)`` re-classes every ``BaselineSelfAttention`` child in
   place (the ``layer.attention.__class__ = ...`` idiom of Project/kernels/k001_sdpa.py:55-61
   and k002_fused_qkv.py:67-72); parameters, names and state-dict keys are untouched.
2. plugin        — ``build(otb, config) -> nn.Module`` (Project/harness/candidate_worker.py:
   275-294): ``otb`` is the official benchmark module; the returned model accepts the
   baseline's state dict with ``strict=True``.
3. model class   — ``make_user_optimized_transformer(otb)`` returns a subclass of
   ``otb.BaselineTransformer`` that swaps its attention modules on construction, the role of
   ``UserOptimizedTransformer`` (torch_transformer_benchmark.py:175-200).
"""
from __future__ import annotations

import torch.nn as nn

from .attention import Int8SelfAttention, SelfAttention

_ATTN_ATTRS = ("d_model", "num_heads", "head_dim", "scale", "q_proj", "k_proj", "v_proj", "out_proj")


def _is_attention(mod: nn.Module) -> bool:
    return all(hasattr(mod, a) for a in _ATTN_ATTRS) and isinstance(getattr(mod, "q_proj"), nn.Linear)


def swap_attention(model: nn.Module, int8: bool = False) -> int:
    """Re-class every attention child of ``model`` in place; returns how many were swapped."""
    cls = Int8SelfAttention if int8 else SelfAttention
    swapped = 0
    for mod in list(model.modules()):
        if _is_attention(mod) and type(mod) is not cls:
            mod.__class__ = cls
            mod.invalidate_caches()
            swapped += 1
    return swapped


def build(otb, config, int8: bool = False) -> nn.Module:
    """Plugin contract of the reference harness: a model whose attention runs on gfx950."""
    base = getattr(otb, "UserOptimizedTransformer", None) or otb.BaselineTransformer
    model = base(config)
    if swap_attention(model, int8=int8) == 0:
        raise RuntimeError("no attention module found to replace")
    return model


def make_user_optimized_transformer(otb, int8: bool = False):
    """A ``UserOptimizedTransformer`` class for the official script module ``otb``."""

    class UserOptimizedTransformer(otb.BaselineTransformer):
        def __init__(self, config):
            super().__init__(config)
            swap_attention(self, int8=int8)

    return UserOptimizedTransformer
