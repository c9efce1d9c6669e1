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

Each takes a scope: the attention module only (default), ``fuse_block`` (each block's attention
half -- norm1, attention, residual -- on the kernels, the FFN half left to torch) or
``full_model`` (every block and the final norm on the kernels, transformer.py).
"""
from __future__ import annotations

import torch.nn as nn
import torch.nn.functional as F

from .attention import Int8SelfAttention, SelfAttention
from .transformer import block_forward, final_norm_forward

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


_BLOCK_ATTRS = ("norm1", "attention", "norm2", "ffn_in", "ffn_out")
_FUSED_CLASSES: dict = {}


def _fused_block_forward(self, x, valid_token_mask, causal):
    """BaselineTransformerBlock.forward (torch_transformer_benchmark.py:134-146) with its attention
    half -- ``x + attention(norm1(x))`` -- on the gfx950 kernels (LayerNorm kernel, fused residual
    epilogue); the FFN half is the reference's own code."""
    x = self.attention.forward_residual(x, self.norm1, valid_token_mask, causal)
    x = x + self.ffn_out(F.gelu(self.ffn_in(self.norm2(x)), approximate="none"))
    if valid_token_mask is not None:
        x = x.masked_fill(~valid_token_mask[..., None], 0)
    return x


def _fused_class(cls):
    if cls not in _FUSED_CLASSES:
        _FUSED_CLASSES[cls] = type("Fused" + cls.__name__, (cls,), {"forward": _fused_block_forward})
    return _FUSED_CLASSES[cls]


def _set_attention_class(mod: nn.Module, int8: bool) -> None:
    cls = Int8SelfAttention if int8 else SelfAttention
    if type(mod.attention) is not cls:
        mod.attention.__class__ = cls
        mod.attention.invalidate_caches()


def swap_blocks(model: nn.Module, int8: bool = False) -> int:
    """Re-class every transformer block of ``model`` (modules with norm1 / attention / norm2 /
    ffn_in / ffn_out) so its attention half runs fused, and its attention on gfx950 (the W8A8
    attention of k008_int8_gemm.py:189-225 with ``int8``); returns how many blocks were swapped.
    Parameters and state-dict keys are untouched."""
    swapped = 0
    for mod in list(model.modules()):
        if all(hasattr(mod, a) for a in _BLOCK_ATTRS) and _is_attention(mod.attention):
            _set_attention_class(mod, int8)
            if type(mod) not in _FUSED_CLASSES.values():
                mod.__class__ = _fused_class(type(mod))
            swapped += 1
    return swapped


_FULL_CLASSES: dict = {}


def _full_block_class(cls):
    if cls not in _FULL_CLASSES:
        _FULL_CLASSES[cls] = type("Kernel" + cls.__name__, (cls,), {"forward": block_forward})
    return _FULL_CLASSES[cls]


def _full_model_forward(self, x, valid_token_mask=None):
    """BaselineTransformer.forward (torch_transformer_benchmark.py:160-172): the (swapped)
    blocks, then final_norm + masked_fill as one masked LayerNorm launch."""
    for layer in self.layers:
        x = layer(x, valid_token_mask, self.config.causal)
    return final_norm_forward(self.final_norm, x, valid_token_mask)


def swap_model(model: nn.Module, int8: bool = False) -> int:
    """Re-class every block of ``model`` so its whole forward runs on the gfx950 kernels
    (transformer.block_forward; with ``int8`` the W8A8 block of k008_int8_gemm.py:189-234) and,
    when ``model`` has ``layers`` / ``final_norm`` / ``config``, the model itself so the final
    norm and its row mask do too; returns how many blocks were swapped. Parameters and
    state-dict keys are untouched."""
    swapped = 0
    for mod in list(model.modules()):
        if all(hasattr(mod, a) for a in _BLOCK_ATTRS) and _is_attention(mod.attention):
            _set_attention_class(mod, int8)
            base = type(mod)
            if base in _FUSED_CLASSES.values():
                base = base.__mro__[1]
            if base not in _FULL_CLASSES.values():
                mod.__class__ = _full_block_class(base)
            swapped += 1
    if swapped and all(hasattr(model, a) for a in ("layers", "final_norm", "config")):
        cls = type(model)
        if not getattr(cls, "_mi355_full_model", False):
            model.__class__ = type("Kernel" + cls.__name__, (cls,),
                                   {"forward": _full_model_forward, "_mi355_full_model": True})
    return swapped


def build(otb, config, int8: bool = False, fuse_block: bool = False,
          full_model: bool = False) -> nn.Module:
    """Plugin contract of the reference harness: a model whose attention runs on gfx950.

    ``fuse_block`` also runs each block's attention half (norm1, attention, residual add) as
    LayerNorm kernel + attention + out projection with the residual fused into its epilogue;
    ``full_model`` runs every block and the final norm on the kernels. ``int8`` selects the W8A8
    recipe of k008_int8_gemm.py (attention projections; with ``full_model`` the FFN too)."""
    base = getattr(otb, "UserOptimizedTransformer", None) or otb.BaselineTransformer
    model = base(config)
    if swap_attention(model, int8=int8) == 0:
        raise RuntimeError("no attention module found to replace")
    if full_model:
        if swap_model(model, int8=int8) == 0:
            raise RuntimeError("no transformer block found to swap")
    elif fuse_block and swap_blocks(model, int8=int8) == 0:
        raise RuntimeError("no transformer block found to fuse")
    return model


def make_user_optimized_transformer(otb, int8: bool = False, fuse_block: bool = False,
                                    full_model: bool = False):
    """A ``UserOptimizedTransformer`` class for the official script module ``otb``."""

    class UserOptimizedTransformer(otb.BaselineTransformer):
        def __init__(self, config):
            super().__init__(config)
            swap_attention(self, int8=int8)
            if fuse_block and not full_model:
                swap_blocks(self, int8=int8)
            if full_model:
                for mod in list(self.modules()):
                    if all(hasattr(mod, a) for a in _BLOCK_ATTRS) and _is_attention(mod.attention):
                        if type(mod) not in _FULL_CLASSES.values():
                            mod.__class__ = _full_block_class(type(mod))

        def forward(self, x, valid_token_mask=None):
            if full_model:
                return _full_model_forward(self, x, valid_token_mask)
            return super().forward(x, valid_token_mask)

    return UserOptimizedTransformer
