"""Drop-in attention modules backed by the gfx950 kernels of libmi355attn.so.

``SelfAttention`` mirrors ``BaselineSelfAttention`` (torch_transformer_benchmark.py:59-122):
same constructor, attributes (d_model, num_heads, head_dim, scale, q_proj, k_proj, v_proj,
out_proj), state-dict keys and ``forward(x, valid_token_mask=None, causal=False)`` contract.
A GPU forward is three launches on the current stream:

  1. packed QKV projection  x[T, d] · W_qkv[3d, d]^T + b_qkv -> qkv[T, 3d]
     (the packing of Project/submission/dispatcher_region.py:789-792);
  2. streamed attention reading q/k/v as strided views of qkv (no head-split copy, as in
     dispatcher_region.py:1026-1029) and writing ctx in [B, S, H, hd] = [T, d] order (the free
     head merge of dispatcher_region.py:314-317);
  3. output projection ctx · W_o^T + b_o with the output-row mask fused in its epilogue.

``Int8SelfAttention`` is the W8A8 variant of Project/kernels/k008_int8_gemm.py:148-235:
per-token int8 activations, per-output-channel int8 weights, exact int32 accumulation, fp32
dequantisation, fp16 SDPA.

Precision policy: fp16 inputs run fp16 storage with fp32 accumulation; bf16 inputs run the
QKV projection on bf16 operands but store q/k/v, the probabilities and the context in fp16
(``bf16_core_dtype``), whose 3 extra mantissa bits keep the block within the elementwise
2e-3 / 2e-2 tolerance of fp32 math that a bf16-stored core misses; the output is bf16. fp32
inputs run the QKV projection in fp32 and, at head dims 32 / 64 / 128, store q/k/v, the
probabilities and the context in fp16 (``fp32_core_dtype``: the fp16 tiles of the reference's
fp32 fast route) so attention runs on the matrix cores; the out projection reads that context
and returns fp32. Other fp32 head dims, and ``fp32_core_dtype = torch.float32``, keep fp32 end
to end. Values beyond the fp16 range (65504) in q/k/v or the context become inf and surface as
non-finite outputs; set the core dtype attributes to the input dtype for such models.

There is no CPU or eager-torch fallback: CPU inputs raise, and a missing library raises.
Derived caches (packed / quantised weights) live in the instance ``__dict__`` and are dropped
on ``load_state_dict`` and ``_apply`` (the contract of dispatcher_region.py:809-836), and are
also re-derived whenever a parameter's storage or version counter changes.
"""
from __future__ import annotations

from typing import Callable, Optional, Tuple

import torch
import torch.nn as nn

from . import ops
from .graph import AutoGraph, version_of

_CACHE_KEYS = ("_mi355_pack", "_mi355_lnpack")

# head dims of the fp16 / bf16 matrix-core attention kernel (the others run on vector ALUs)
MFMA_HEAD_DIMS = (32, 64, 128)


def norm_stamp(norm: nn.Module) -> Tuple:
    """Identity of a LayerNorm's parameters (storage, version, dtype, device) and eps."""
    return tuple((p.data_ptr(), version_of(p), p.dtype, p.device) if p is not None else None
                 for p in (norm.weight, norm.bias)) + (float(norm.eps),)


class SelfAttention(nn.Module):
    """Multi-head self-attention with the reference's module API, on gfx950 kernels."""

    bf16_core_dtype = torch.float16
    # fp32 models at the matrix-core head dims (32, 64, 128) keep the projections' operands in
    # fp32 but carry q/k/v, the probabilities and the context in fp16, so attention runs on the
    # fp16 MFMA kernel -- the fp16 tiles the reference's fast route uses for fp32 models
    # (Project/submission/dispatcher_region.py:1017-1091); the out projection reads the fp16
    # context with an fp16 copy of its weight and returns fp32. torch.float32 keeps the core
    # in fp32 (the vector-ALU kernel).
    fp32_core_dtype = torch.float16
    # forward_residual folds the LayerNorm into the QKV projection (row statistics pass + the
    # projection's epilogue) for fp32 and fp16 inputs; False runs the LayerNorm kernel and a
    # plain projection instead
    fold_norm = True

    # the attention kernel's key-norm bound workspace (ops.attention): None = the library's
    # choice (long key ranges: the max-free and offset sweeps) and the causal policy below,
    # True = at every length, False = the exact running max
    key_bound: Optional[bool] = None
    # causal calls from this many keys on take the key-norm bounds -- written by the QKV
    # projection's epilogue where its shapes allow (same bits as the attention's bound pass,
    # which runs otherwise) -- and their query tiles from this key range on take the max-free /
    # offset sweeps (head_dim 32 / 64; C3, causal S 8192: +7% attention). A prefix run gives
    # the full run's rows bit for bit as long as both lengths are on the same side of it.
    causal_sweep_min_keys = 2048
    # non-causal calls below the library's recommended length take the bounds when the QKV
    # projection can write them (C2: +3.5% attention, the offset sweep at 2^11)
    noncausal_projection_bounds = True
    # fp32 models whose core is fp16 (the matrix-core head dims): the block's projections take
    # fp16 operands too -- the LayerNorms compute in fp32 and write fp16, the weights are packed
    # in fp16, accumulation and the residual stream stay fp32 -- as the reference's fast route
    # runs fp32 models on fp16 tiles (Project/submission/dispatcher_region.py:1017-1091);
    # torch.float32 keeps fp32 operands (the LayerNorms then folded into the projections)
    fp32_operand_dtype = torch.float16
    # ... from this many input elements on (0: always). The fp16 projections take tiles sized to
    # the problem (128 x 128 / 64 x 64 on small ones), so they beat the fp32 path (LayerNorm
    # folded into 128 x 128-tile fp32 projections) at every size measured: official shapes 1, 5,
    # 9, 10 (8192-16384 tokens of 128 features) 0.34-0.41 -> 0.21-0.30 ms per forward, shapes
    # 2-4 and 12 8-12% faster. (With 256 x 256 fp16 tiles only, the fp32 path had been faster
    # below 2^23 elements.)
    fp16_operand_min_elems = 0

    def operand_dtype(self, dtype: torch.dtype, numel: int = 1 << 62) -> torch.dtype:
        """Operand dtype of the block's projections (forward_residual, the FFN half) for model
        dtype ``dtype`` and an input of ``numel`` elements."""
        if (dtype == torch.float32 and self.core_dtype(dtype) == torch.float16
                and numel >= self.fp16_operand_min_elems):
            return self.fp32_operand_dtype
        return dtype

    def folds_norm(self, dtype: torch.dtype, numel: int = 1 << 62) -> bool:
        """Whether forward_residual (and the block's FFN half) fold the LayerNorm for inputs of
        ``dtype``. bf16 keeps the LayerNorm kernel: the fold rounds gamma * W to bf16 where the
        reference rounds the normalised activations, and at bf16's 8-bit precision that moves
        about one output in 10^4 by a bf16 step beyond the reference's own rounding points.
        fp32 models on fp16 operands also run the LayerNorm kernel (fp32 statistics, fp16
        output): folding would round the raw x to fp16, whose mean need not be small."""
        return (bool(self.fold_norm) and dtype != torch.bfloat16
                and self.operand_dtype(dtype, numel) == dtype)

    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__()
        if d_model % num_heads != 0:
            raise ValueError("d_model must be divisible by num_heads")
        self.d_model = d_model
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.scale = self.head_dim ** -0.5
        self.q_proj = nn.Linear(d_model, d_model, bias=True)
        self.k_proj = nn.Linear(d_model, d_model, bias=True)
        self.v_proj = nn.Linear(d_model, d_model, bias=True)
        self.out_proj = nn.Linear(d_model, d_model, bias=True)

    # ----------------------------------------------------------------------------- caches
    def invalidate_caches(self) -> None:
        for key in _CACHE_KEYS:
            self.__dict__.pop(key, None)

    def load_state_dict(self, *args, **kwargs):
        result = super().load_state_dict(*args, **kwargs)
        self.invalidate_caches()
        return result

    def _apply(self, fn, recurse=True):
        result = super()._apply(fn, recurse=recurse)
        self.invalidate_caches()
        return result

    def _param_stamp(self) -> Tuple:
        stamp = []
        for lin in (self.q_proj, self.k_proj, self.v_proj, self.out_proj):
            for p in (lin.weight, lin.bias):
                stamp.append((p.data_ptr(), version_of(p), p.dtype, p.device))
        return tuple(stamp)

    def _cached(self, key, build):
        entry = self.__dict__.get("_mi355_pack")
        if entry is not None and entry[0] == key:
            return entry[1]
        value = build()
        self.__dict__["_mi355_pack"] = (key, value)
        return value

    def core_dtype(self, dtype: torch.dtype) -> torch.dtype:
        """Storage dtype of q/k/v, probabilities and context for input dtype ``dtype``."""
        if dtype == torch.bfloat16:
            return self.bf16_core_dtype
        if dtype == torch.float32 and self.head_dim in MFMA_HEAD_DIMS:
            return self.fp32_core_dtype
        return dtype

    def _packed_weights(self, dtype: torch.dtype, device: torch.device):
        """(W_qkv [3d, d] in the input dtype, b_qkv fp32, W_o [d, d] in the core dtype, b_o fp32)."""
        core = self.core_dtype(dtype)

        def build():
            with torch.no_grad():
                w_qkv = torch.cat([self.q_proj.weight, self.k_proj.weight, self.v_proj.weight], 0)
                b_qkv = torch.cat([self.q_proj.bias, self.k_proj.bias, self.v_proj.bias], 0)
                f32 = torch.float32
                return (w_qkv.to(device=device, dtype=dtype).contiguous(),
                        b_qkv.to(device=device, dtype=f32).contiguous(),
                        self.out_proj.weight.to(device=device, dtype=core).contiguous(),
                        self.out_proj.bias.to(device=device, dtype=f32).contiguous())
        return self._cached(("fp", dtype, core, device, self._param_stamp()), build)

    def _ln_folded_qkv(self, norm: nn.LayerNorm, dtype: torch.dtype, device: torch.device):
        """(Wf [3d, d] in dtype, colsum [3d] fp32, bias' [3d] fp32): ``norm`` folded into the
        packed QKV projection (ops.fold_layernorm), cached beside the packed weights."""
        key = ("ln", dtype, device, self._param_stamp(), norm_stamp(norm))
        entry = self.__dict__.get("_mi355_lnpack")
        if entry is not None and entry[0] == key:
            return entry[1]
        with torch.no_grad():
            w_qkv = torch.cat([self.q_proj.weight, self.k_proj.weight, self.v_proj.weight], 0)
            b_qkv = torch.cat([self.q_proj.bias, self.k_proj.bias, self.v_proj.bias], 0)
            value = ops.fold_layernorm(w_qkv.to(device), b_qkv.to(device), norm.weight, norm.bias,
                                       dtype)
        self.__dict__["_mi355_lnpack"] = (key, value)
        return value

    # ------------------------------------------------------------------------------- masks
    def _resolve_mask(self, mask: Optional[torch.Tensor], B: int, S: int, device: torch.device):
        """Returns (key_valid [B,S] bool or None, row_valid [B*S] bool or None).

        A given mask goes to the kernels as it is; nothing is decided on the host. The attention
        kernel checks each work-group's mask bytes on the device and masks element-wise only
        where a tile holds invalid keys; with the key-norm bound workspace (long key ranges) the
        bound pass marks the chunks that hold invalid keys, the unmasked kernel (max-free and
        offset sweeps) runs every work-group whose keys are all valid and a second, key-masked
        launch runs the rest. An all-true mask therefore costs about what no mask costs, and the
        forward never synchronises the host (eager and captured calls take the same kernels).
        """
        if mask is None:
            return None, None
        if mask.dtype != torch.bool or tuple(mask.shape) != (B, S):
            raise ValueError(f"valid_token_mask must be a bool tensor of shape ({B}, {S})")
        if mask.device != device:
            raise ValueError("valid_token_mask must be on the input's device")
        m = mask if mask.is_contiguous() else mask.contiguous()
        return m, m.view(B * S)

    # ----------------------------------------------------------------------------- forward
    def _check_input(self, x: torch.Tensor) -> Tuple[int, int]:
        if x.dim() != 3 or x.shape[-1] != self.d_model:
            raise ValueError(f"expected x of shape [B, S, {self.d_model}], got {tuple(x.shape)}")
        if x.device.type != "cuda":
            raise RuntimeError("SelfAttention runs only on the GPU kernels; got a "
                               f"{x.device.type} tensor (there is no CPU path)")
        if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            raise TypeError(f"unsupported dtype {x.dtype}")
        return x.shape[0], x.shape[1]

    def _bound_plan(self, B: int, S: int, core: torch.dtype, causal: bool,
                    key_valid: Optional[torch.Tensor],
                    device: torch.device) -> Optional[ops.KeyBoundTarget]:
        """Where this forward's key-norm bounds go (``key_bound``, ``causal_sweep_min_keys``,
        ``noncausal_projection_bounds``), or None to leave the choice to ``ops.attention``."""
        kb, hd = self.key_bound, self.head_dim
        if kb is False or core not in (torch.float16, torch.bfloat16) or hd not in (32, 64, 128):
            return None
        if kb is None:
            if hd == 128:  # no sweep pays there (the offset sweep's estimate fails)
                return None
            if causal and S < self.causal_sweep_min_keys:
                return None
            if not causal and not self.noncausal_projection_bounds:
                return None
        ws = ops.attention_workspace(B, S, S, self.num_heads, hd, core, device)
        if ws.numel() == 0:
            return None
        return ops.KeyBoundTarget(ws, k_col0=self.d_model, heads=self.num_heads, head_dim=hd,
                                  seq=S, key_valid=key_valid)

    def _attend(self, q, k, v, causal: bool, key_valid: Optional[torch.Tensor],
                kbt: Optional[ops.KeyBoundTarget]) -> torch.Tensor:
        if kbt is not None and (kbt.written or causal or self.key_bound):
            return ops.attention(q, k, v, scale=self.scale, causal=causal, key_valid=key_valid,
                                 workspace=kbt.workspace, bounds_ready=kbt.written,
                                 causal_sweep_min_keys=self.causal_sweep_min_keys)
        return ops.attention(q, k, v, scale=self.scale, causal=causal, key_valid=key_valid,
                             key_bound=self.key_bound)

    def _qkv_views(self, qkv: torch.Tensor, B: int, S: int):
        qkv5 = qkv.view(B, S, 3, self.num_heads, self.head_dim)
        return qkv5[:, :, 0], qkv5[:, :, 1], qkv5[:, :, 2]

    # launch-bound forwards (small inputs, inference) replay a captured graph (graph.AutoGraph)
    auto_graph = True
    # attributes the forward reads besides parameters: a captured graph (graph.AutoGraph) is
    # recorded again when one of them changes
    graph_switches = ("bf16_core_dtype", "fp32_core_dtype", "fold_norm", "key_bound",
                      "causal_sweep_min_keys", "noncausal_projection_bounds",
                      "fp32_operand_dtype", "fp16_operand_min_elems")

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None,
                causal: bool = False) -> torch.Tensor:
        if self.auto_graph:
            ag = self.__dict__.get("_autograph")
            if ag is None:
                ag = self.__dict__["_autograph"] = AutoGraph()
            out = ag(self, lambda sx, sm: self.run(sx, sm, causal), x, valid_token_mask,
                     (bool(causal),))
            if out is not None:
                return out
        return self.run(x, valid_token_mask, causal)

    def run(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None,
            causal: bool = False, keep: Optional[dict] = None,
            marks: Optional[Callable[[str], None]] = None) -> torch.Tensor:
        """The forward pass.

        ``keep`` (a dict) receives the qkv and ctx intermediates; ``marks(stage)`` is called
        before each kernel launch ("qkv", "attn", "out") and after the last ("end"), so a caller
        can bracket every kernel with events on the launch stream.
        """
        mark = marks or (lambda _stage: None)
        B, S = self._check_input(x)
        d = self.d_model
        key_valid, row_valid = self._resolve_mask(valid_token_mask, B, S, x.device)
        w_qkv, b_qkv, w_o, b_o = self._packed_weights(x.dtype, x.device)
        core = self.core_dtype(x.dtype)
        x2 = x.reshape(B * S, d)
        if x2.stride(1) != 1:
            x2 = x2.contiguous()
        kbt = self._bound_plan(B, S, core, causal, key_valid, x.device)
        mark("qkv")
        qkv = ops.linear(x2, w_qkv, b_qkv, out_dtype=core, key_bounds=kbt)
        q, k, v = self._qkv_views(qkv, B, S)
        mark("attn")
        ctx = self._attend(q, k, v, causal, key_valid, kbt)
        mark("out")
        out = ops.linear(ctx.view(B * S, d), w_o, b_o, row_valid=row_valid, out_dtype=x.dtype)
        mark("end")
        if keep is not None:
            keep.update(qkv=qkv, ctx=ctx)
        return out.view(B, S, d)

    def forward_residual(self, x: torch.Tensor, norm: nn.LayerNorm,
                         valid_token_mask: Optional[torch.Tensor] = None, causal: bool = False,
                         marks: Optional[Callable[[str], None]] = None) -> torch.Tensor:
        """``x + self(norm(x), valid_token_mask, causal)``: the attention half of
        BaselineTransformerBlock.forward (torch_transformer_benchmark.py:139).

        For fp16 inputs (and fp32 inputs on fp32 projection operands) the LayerNorm is folded
        into the QKV projection (``fold_norm``, ``folds_norm``; the reference's fused
        LN-prologue QKV kernels Project/kernels/k024_cuda_tuned.py:94-197 and
        Project/submission/dispatcher_region.py:343-399): a row-statistics pass, then the
        projection of the raw x with gamma folded into the weights and the mean / rstd / beta
        applied in its epilogue, so the normalised rows are never written. With
        ``fold_norm = False``, for bf16 and for fp32 inputs on fp16 operands it runs as its own
        row kernel (fp32 statistics, rounded to x's dtype as nn.LayerNorm's output is, or to the
        fp16 operand type). The residual add is fused into the out projection's
        epilogue, where the projection is rounded to x's dtype before the add, as in the
        reference; rows masked out keep x. ``marks`` as for ``run``; the unfolded form has an
        extra "norm" stage before "qkv".
        """
        mark = marks or (lambda _stage: None)
        B, S = self._check_input(x)
        d = self.d_model
        if tuple(norm.normalized_shape) != (d,):
            raise ValueError(f"norm must normalise the last dimension ({d})")
        w_n, b_n = norm.weight, norm.bias
        for t in (w_n, b_n):
            if t is not None and (t.dtype != x.dtype or t.device != x.device):
                raise ValueError("norm parameters must be on x's device in x's dtype")
        key_valid, row_valid = self._resolve_mask(valid_token_mask, B, S, x.device)
        op = self.operand_dtype(x.dtype, x.numel())
        w_qkv, b_qkv, w_o, b_o = self._packed_weights(op, x.device)
        core = self.core_dtype(x.dtype)
        x2 = x.reshape(B * S, d)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        kbt = self._bound_plan(B, S, core, causal, key_valid, x.device)
        if self.folds_norm(x.dtype, x.numel()):
            wf, colsum, bf = self._ln_folded_qkv(norm, x.dtype, x.device)
            mark("qkv")
            qkv = ops.layernorm_linear(x2, wf, colsum, bf, norm.eps, out_dtype=core,
                                       key_bounds=kbt)
        else:
            mark("norm")
            h = ops.layer_norm(x2, w_n.detach() if w_n is not None else None,
                               b_n.detach() if b_n is not None else None, norm.eps, out_dtype=op)
            mark("qkv")
            qkv = ops.linear(h, w_qkv, b_qkv, out_dtype=core, key_bounds=kbt)
        q, k, v = self._qkv_views(qkv, B, S)
        mark("attn")
        ctx = self._attend(q, k, v, causal, key_valid, kbt)
        mark("out")
        out = ops.linear(ctx.view(B * S, d), w_o, b_o, row_valid=row_valid, out_dtype=x.dtype,
                         residual=x2)
        mark("end")
        return out.view(B, S, d)


class Int8SelfAttention(SelfAttention):
    """W8A8 variant: int8 projections with exact int32 accumulation, fp16 SDPA.

    Mirrors the attention half of ``block_forward`` in Project/kernels/k008_int8_gemm.py:189-225:
    qkv = fp16(int8_linear(x)) -> fp16 attention -> int8_linear(ctx). The output dtype is the
    input dtype.
    """

    def _int8_weights(self, device: torch.device):
        def build():
            with torch.no_grad():
                w_qkv = torch.cat([self.q_proj.weight, self.k_proj.weight, self.v_proj.weight], 0)
                b_qkv = torch.cat([self.q_proj.bias, self.k_proj.bias, self.v_proj.bias], 0)
                w_qkv = w_qkv.to(device=device, dtype=torch.float32).contiguous()
                w_o = self.out_proj.weight.to(device=device, dtype=torch.float32).contiguous()
                wq_i8, s_qkv = ops.quant_rows_i8(w_qkv, mode=1)
                wo_i8, s_o = ops.quant_rows_i8(w_o, mode=1)
                return (wq_i8, s_qkv, b_qkv.to(device=device, dtype=torch.float32).contiguous(),
                        wo_i8, s_o,
                        self.out_proj.bias.to(device=device, dtype=torch.float32).contiguous())
        return self._cached(("i8", device, self._param_stamp()), build)

    def run(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None,
            causal: bool = False, keep: Optional[dict] = None,
            marks: Optional[Callable[[str], None]] = None) -> torch.Tensor:
        mark = marks or (lambda _stage: None)
        B, S = self._check_input(x)
        d = self.d_model
        if d % 16:
            raise ValueError("the int8 path needs d_model % 16 == 0")
        key_valid, row_valid = self._resolve_mask(valid_token_mask, B, S, x.device)
        wq, s_qkv, b_qkv, wo, s_o, b_o = self._int8_weights(x.device)
        x2 = x.reshape(B * S, d)
        if x2.stride(1) != 1:
            x2 = x2.contiguous()
        mark("quant_x")
        xq, sx = ops.quant_rows_i8(x2, mode=0)
        mark("qkv")
        qkv = ops.linear_i8(xq, wq, sx, s_qkv, b_qkv, out_dtype=torch.float16)
        q, k, v = self._qkv_views(qkv, B, S)
        mark("attn")
        ctx = ops.attention(q, k, v, scale=self.scale, causal=causal, key_valid=key_valid,
                                key_bound=self.key_bound)
        mark("quant_ctx")
        cq, sc = ops.quant_rows_i8(ctx.view(B * S, d), mode=0)
        mark("out")
        out = ops.linear_i8(cq, wo, sc, s_o, b_o, out_dtype=x.dtype, row_valid=row_valid)
        mark("end")
        if keep is not None:
            keep.update(qkv=qkv, ctx=ctx, x_i8=xq, x_scale=sx, ctx_i8=cq, ctx_scale=sc)
        return out.view(B, S, d)

    def forward_residual(self, x: torch.Tensor, norm: nn.LayerNorm,
                         valid_token_mask: Optional[torch.Tensor] = None, causal: bool = False,
                         marks: Optional[Callable[[str], None]] = None,
                         keep: Optional[dict] = None) -> torch.Tensor:
        """The attention half of the int8 block (block_forward,
        Project/kernels/k008_int8_gemm.py:189-225): h = norm1(x) (LayerNorm kernel), W8A8 QKV to
        fp16, fp16 attention, W8A8 out projection with ``x + attn_out`` fused into its epilogue
        (masked rows keep x, :221-225). ``marks`` as for ``run`` with an extra "norm" stage;
        ``keep`` (a dict) receives the intermediates."""
        mark = marks or (lambda _stage: None)
        B, S = self._check_input(x)
        d = self.d_model
        if d % 16:
            raise ValueError("the int8 path needs d_model % 16 == 0")
        if tuple(norm.normalized_shape) != (d,):
            raise ValueError(f"norm must normalise the last dimension ({d})")
        w_n, b_n = norm.weight, norm.bias
        for t in (w_n, b_n):
            if t is not None and (t.dtype != x.dtype or t.device != x.device):
                raise ValueError("norm parameters must be on x's device in x's dtype")
        key_valid, row_valid = self._resolve_mask(valid_token_mask, B, S, x.device)
        wq, s_qkv, b_qkv, wo, s_o, b_o = self._int8_weights(x.device)
        x2 = x.reshape(B * S, d)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        mark("norm")
        h = ops.layer_norm(x2, w_n.detach() if w_n is not None else None,
                           b_n.detach() if b_n is not None else None, norm.eps)
        mark("quant_x")
        hq, sh = ops.quant_rows_i8(h, mode=0)
        mark("qkv")
        qkv = ops.linear_i8(hq, wq, sh, s_qkv, b_qkv, out_dtype=torch.float16)
        q, k, v = self._qkv_views(qkv, B, S)
        mark("attn")
        ctx = ops.attention(q, k, v, scale=self.scale, causal=causal, key_valid=key_valid,
                                key_bound=self.key_bound)
        mark("quant_ctx")
        cq, sc = ops.quant_rows_i8(ctx.view(B * S, d), mode=0)
        mark("out")
        out = ops.linear_i8(cq, wo, sc, s_o, b_o, out_dtype=x.dtype, row_valid=row_valid,
                            residual=x2)
        mark("end")
        if keep is not None:
            keep.update(h=h, h_i8=hq, h_scale=sh, qkv=qkv, ctx=ctx, ctx_i8=cq, ctx_scale=sc)
        return out.view(B, S, d)
