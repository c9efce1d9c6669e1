"""The benchmark's whole transformer on the gfx950 kernels of libmi355attn.so.

``TransformerBlock`` mirrors ``BaselineTransformerBlock`` (torch_transformer_benchmark.py:125-145)
and ``Transformer`` mirrors ``BaselineTransformer`` / ``UserOptimizedTransformer`` (:148-200):
same constructor arguments, attribute and parameter names (so a baseline state dict loads with
``strict=True``) and forward signatures. A block forward is seven launches on the current stream:

  1. norm1 statistics + packed QKV projection with norm1 folded in
                                          qkv = norm1(x) W_qkv^T + b_qkv        (:139, :93-95)
  2. streamed attention                   ctx                                  (:97-117)
  3. out projection + residual epilogue   x1 = x + out_proj(ctx), masked rows x (:118-121, :139)
  4. norm2 statistics + ffn_in with norm2 folded in and the GELU epilogue
                                          g = gelu(ffn_in(norm2(x1)))          (:141)
  5. ffn_out + residual + row-mask epilogue  y = x1 + ffn_out(g), masked rows 0  (:141-144)

(1 and 4 are two launches each: a row-statistics pass and the projection, whose epilogue applies
the mean, rstd and beta; gamma is folded into the weights. bf16 models, and
``SelfAttention.fold_norm = False``, run the LayerNorms as their own row kernels instead.)

and the model adds one masked LayerNorm launch for ``final_norm`` + masked_fill (:168-171).
Every rounding point of the reference's dtype arithmetic is kept: each nn.Linear output is
rounded to the model dtype before GELU / the residual add, and each sum is rounded again.
fp32, fp16 and bf16 models are supported (bf16 attention cores run in fp16, see
``SelfAttention.bf16_core_dtype``). A block whose attention is an ``Int8SelfAttention`` runs the
int8 block of Project/kernels/k008_int8_gemm.py:189-234 instead: all four projections W8A8
(per-token activation scales from the quantisation kernel, per-channel weight scales), each
projection input quantised by one extra launch, GELU and both residual adds fused into the int8
GEMM epilogues. There is no CPU path: CPU inputs raise.
"""
from __future__ import annotations

from typing import Callable, Optional

import torch
import torch.nn as nn

from . import ops
from .attention import Int8SelfAttention, SelfAttention
from .graph import AutoGraph, version_of


def _stamp(*params):
    return tuple((p.data_ptr(), version_of(p), p.dtype, p.device) for p in params if p is not None)


def _ffn_weights(block: nn.Module, dtype: torch.dtype, device: torch.device):
    """(W_in [ffn, d], b_in fp32, W_out [d, ffn], b_out fp32) in the model dtype, cached on the
    block and re-derived when a parameter's storage or version changes."""
    key = ("ffn", dtype, device, _stamp(block.ffn_in.weight, block.ffn_in.bias,
                                        block.ffn_out.weight, block.ffn_out.bias))
    entry = block.__dict__.get("_mi355_ffn")
    if entry is not None and entry[0] == key:
        return entry[1]
    with torch.no_grad():
        f32 = torch.float32

        def b(lin):
            if lin.bias is None:
                return None
            return lin.bias.to(device=device, dtype=f32).contiguous()

        value = (block.ffn_in.weight.to(device=device, dtype=dtype).contiguous(), b(block.ffn_in),
                 block.ffn_out.weight.to(device=device, dtype=dtype).contiguous(), b(block.ffn_out))
    block.__dict__["_mi355_ffn"] = (key, value)
    return value


def _ffn_in_folded(block: nn.Module, dtype: torch.dtype, device: torch.device):
    """(Wf [ffn, d] in dtype, colsum fp32, bias' fp32): norm2 folded into ffn_in
    (ops.fold_layernorm), cached on the block like ``_ffn_weights``."""
    n2 = block.norm2
    key = ("ffn_in_ln", dtype, device, _stamp(block.ffn_in.weight, block.ffn_in.bias, n2.weight,
                                              n2.bias), float(n2.eps))
    entry = block.__dict__.get("_mi355_ffn_ln")
    if entry is not None and entry[0] == key:
        return entry[1]
    with torch.no_grad():
        w = block.ffn_in.weight.to(device=device)
        b = None if block.ffn_in.bias is None else block.ffn_in.bias.to(device=device)
        value = ops.fold_layernorm(w, b, n2.weight, n2.bias, dtype)
    block.__dict__["_mi355_ffn_ln"] = (key, value)
    return value


def _ffn_weights_i8(block: nn.Module, device: torch.device):
    """(W_in int8 [ffn, d], s_in, b_in, W_out int8 [d, ffn], s_out, b_out): the weight recipe of
    ``_int8_pack`` (k008_int8_gemm.py:154-158) applied by the quantisation kernel to the fp32
    weights, cached on the block like ``_ffn_weights``."""
    key = ("ffn_i8", device, _stamp(block.ffn_in.weight, block.ffn_in.bias,
                                    block.ffn_out.weight, block.ffn_out.bias))
    entry = block.__dict__.get("_mi355_ffn_i8")
    if entry is not None and entry[0] == key:
        return entry[1]
    with torch.no_grad():
        f32 = torch.float32

        def pack(lin):
            w = lin.weight.to(device=device, dtype=f32).contiguous()
            w_i8, s_w = ops.quant_rows_i8(w, mode=1)
            b = None if lin.bias is None else lin.bias.to(device=device, dtype=f32).contiguous()
            return w_i8, s_w, b

        value = pack(block.ffn_in) + pack(block.ffn_out)
    block.__dict__["_mi355_ffn_i8"] = (key, value)
    return value


def _norm_params(norm: nn.LayerNorm, x: torch.Tensor):
    d = x.shape[-1]
    if tuple(norm.normalized_shape) != (d,):
        raise ValueError(f"LayerNorm must normalise the last dimension ({d})")
    w, b = norm.weight, norm.bias
    for t in (w, b):
        if t is not None and (t.dtype != x.dtype or t.device != x.device):
            raise ValueError("LayerNorm parameters must be on x's device in x's dtype")
    return (w.detach() if w is not None else None), (b.detach() if b is not None else None)


def block_forward(block: nn.Module, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor],
                  causal: bool, marks: Optional[Callable[[str], None]] = None,
                  keep: Optional[dict] = None) -> torch.Tensor:
    """BaselineTransformerBlock.forward (torch_transformer_benchmark.py:134-145) on the gfx950
    kernels, for any module with the block's attributes whose ``attention`` is a SelfAttention
    (or an Int8SelfAttention: the W8A8 block).

    With ``attention.folds_norm(dtype)`` (fp16 models by default) norm1 is folded into the QKV projection and norm2
    into ffn_in (row-statistics pass + projection epilogue, ``ops.layernorm_linear``), so neither
    normalised activation is written. ``marks(stage)`` is called before each launch ("qkv",
    "attn", "out", "ffn_in", "ffn_out"; unfolded, "norm" and "norm2" before the LayerNorm
    kernels; the int8 block adds its quantisation launches) and after the last ("end").
    ``keep`` (a dict) receives the int8 block's intermediates."""
    mark = marks or (lambda _stage: None)
    attn = block.attention
    if not isinstance(attn, SelfAttention):
        raise TypeError("the block's attention must be a SelfAttention or Int8SelfAttention")
    if isinstance(attn, Int8SelfAttention):
        return _block_forward_i8(block, x, valid_token_mask, causal, mark, keep)
    B, S = attn._check_input(x)
    d = attn.d_model
    _, row_valid = attn._resolve_mask(valid_token_mask, B, S, x.device)

    def inner(stage):
        if stage != "end":
            mark(stage)

    x1 = attn.forward_residual(x, block.norm1, valid_token_mask, causal, marks=inner)
    x1 = x1.reshape(B * S, d)
    w2, b2 = _norm_params(block.norm2, x)
    # the FFN's operand dtype: the model's, or fp16 for fp32 models with an fp16 attention core
    # (SelfAttention.operand_dtype; the GELU output is then fp16 too, the residual stream fp32)
    op = attn.operand_dtype(x.dtype, x.numel())
    w_in, b_in, w_out, b_out = _ffn_weights(block, op, x.device)
    if attn.folds_norm(x.dtype, x.numel()):
        wf, colsum, bf = _ffn_in_folded(block, x.dtype, x.device)
        mark("ffn_in")
        g = ops.layernorm_linear(x1, wf, colsum, bf, block.norm2.eps, gelu=True)
    else:
        mark("norm2")
        h2 = ops.layer_norm(x1, w2, b2, block.norm2.eps, out_dtype=op)
        mark("ffn_in")
        g = ops.linear(h2, w_in, b_in, gelu=True, out_dtype=op)
    mark("ffn_out")
    y = ops.linear(g, w_out, b_out, residual=x1, row_valid=row_valid, zero_masked_rows=True,
                   out_dtype=x.dtype)
    mark("end")
    return y.view(B, S, d)


def _block_forward_i8(block: nn.Module, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor],
                      causal: bool, mark: Callable[[str], None],
                      keep: Optional[dict] = None) -> torch.Tensor:
    """The int8 block (block_forward, Project/kernels/k008_int8_gemm.py:189-234): the attention
    half from Int8SelfAttention.forward_residual, then h2 = norm2(x1), g = gelu(int8_linear(h2))
    (:227-229) and y = x1 + int8_linear(g) with masked rows zeroed (:230-233). Every projection
    input is quantised per row by the quantisation kernel (``_quant_rows``, :148-151) from its
    values in x's dtype (fp32 for the benchmark's default models, as in the reference)."""
    attn = block.attention
    B, S = attn._check_input(x)
    d = attn.d_model
    ffn = block.ffn_in.out_features
    if ffn % 16:
        raise ValueError("the int8 FFN needs ffn_dim % 16 == 0")
    _, row_valid = attn._resolve_mask(valid_token_mask, B, S, x.device)

    def inner(stage):
        if stage != "end":
            mark(stage)

    attn_keep = {} if keep is not None else None
    x1 = attn.forward_residual(x, block.norm1, valid_token_mask, causal, marks=inner,
                               keep=attn_keep)
    x1 = x1.reshape(B * S, d)
    w2, b2 = _norm_params(block.norm2, x)
    w_in, s_in, b_in, w_out, s_out, b_out = _ffn_weights_i8(block, x.device)
    mark("norm2")
    h2 = ops.layer_norm(x1, w2, b2, block.norm2.eps)
    mark("quant_h2")
    hq, sh = ops.quant_rows_i8(h2, mode=0)
    mark("ffn_in")
    g = ops.linear_i8(hq, w_in, sh, s_in, b_in, out_dtype=x.dtype, gelu=True)
    mark("quant_g")
    gq, sg = ops.quant_rows_i8(g, mode=0)
    mark("ffn_out")
    y = ops.linear_i8(gq, w_out, sg, s_out, b_out, out_dtype=x.dtype, residual=x1,
                      row_valid=row_valid, zero_masked_rows=True)
    mark("end")
    if keep is not None:
        keep.update(attn_keep)
        keep.update(x1=x1, h2=h2, h2_i8=hq, h2_scale=sh, g=g, g_i8=gq, g_scale=sg)
    return y.view(B, S, d)


def final_norm_forward(norm: nn.LayerNorm, x: torch.Tensor,
                       valid_token_mask: Optional[torch.Tensor]) -> torch.Tensor:
    """``final_norm(x)`` then ``masked_fill(~valid_token_mask[..., None], 0)``
    (torch_transformer_benchmark.py:168-171) as one masked LayerNorm launch."""
    if x.dim() != 3:
        raise ValueError("expected x of shape [B, S, d]")
    B, S, d = x.shape
    if x.device.type != "cuda":
        raise RuntimeError("the transformer runs only on the GPU kernels (no CPU path)")
    row_valid = None
    if valid_token_mask is not None:
        if valid_token_mask.dtype != torch.bool or tuple(valid_token_mask.shape) != (B, S):
            raise ValueError(f"valid_token_mask must be a bool tensor of shape ({B}, {S})")
        row_valid = valid_token_mask.contiguous().view(B * S)
    w, b = _norm_params(norm, x)
    x2 = x.reshape(B * S, d)
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    return ops.layer_norm(x2, w, b, norm.eps, row_valid=row_valid).view(B, S, d)


class TransformerBlock(nn.Module):
    """Pre-LN transformer block with the reference's API (torch_transformer_benchmark.py:125-145)."""

    def __init__(self, d_model: int, num_heads: int, ffn_dim: int, int8: bool = False) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attention = (Int8SelfAttention if int8 else SelfAttention)(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn_in = nn.Linear(d_model, ffn_dim)
        self.ffn_out = nn.Linear(ffn_dim, d_model)

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor],
                causal: bool) -> torch.Tensor:
        return block_forward(self, x, valid_token_mask, causal)


class Transformer(nn.Module):
    """``BaselineTransformer`` with the reference's API (torch_transformer_benchmark.py:148-172).

    ``config`` needs ``d_model``, ``num_heads``, ``ffn_dim``, ``num_layers`` and ``causal``
    (the reference's TransformerConfig, :29-56). ``int8`` builds the W8A8 blocks of
    Project/kernels/k008_int8_gemm.py:189-234 (same parameters; the int8 weights are derived)."""

    def __init__(self, config, int8: bool = False) -> None:
        super().__init__()
        self.config = config
        self.layers = nn.ModuleList(
            [TransformerBlock(config.d_model, config.num_heads, config.ffn_dim, int8=int8)
             for _ in range(config.num_layers)])
        self.final_norm = nn.LayerNorm(config.d_model)

    # launch-bound forwards (small inputs, inference) replay a captured graph (graph.AutoGraph),
    # as the reference's optimised model does (Project/submission/dispatcher_region.py:1220-1363)
    auto_graph = True

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if self.auto_graph:
            ag = self.__dict__.get("_autograph")
            if ag is None:
                ag = self.__dict__["_autograph"] = AutoGraph()
            out = ag(self, self._eager_forward, x, valid_token_mask, (bool(self.config.causal),))
            if out is not None:
                return out
        return self._eager_forward(x, valid_token_mask)

    def _eager_forward(self, x: torch.Tensor,
                       valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        for layer in self.layers:
            x = layer(x, valid_token_mask, self.config.causal)
        return final_norm_forward(self.final_norm, x, valid_token_mask)


UserOptimizedTransformer = Transformer
