"""Torch-facing wrappers of the libmi355attn entry points.

Each wrapper validates shapes/dtypes/devices on the host, allocates outputs with torch (the
library never allocates), and enqueues the kernel on torch's current stream of the tensors'
device. Nothing here synchronises the host, so the calls are hipGraph-capturable.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _lib

# status of an entry point that cannot run the requested combination (nothing launched)
_E_UNSUPPORTED = -6


@dataclass
class KeyBoundTarget:
    """Where a QKV projection writes the attention's key-norm bounds (``mi355_*_kbound``).

    ``workspace`` is the attention workspace (uint8, ``attention_workspace``), whose bound
    section the projection fills for the K block: output columns ``[k_col0, k_col0 + heads *
    head_dim)`` of ``seq`` tokens per batch row, with ``key_valid`` ([B, seq] bool, optional)
    marking chunks that hold an invalid key. ``written`` tells whether the projection wrote
    them (the fused epilogue has shape requirements; otherwise the attention runs its own pass).
    """
    workspace: torch.Tensor
    k_col0: int
    heads: int
    head_dim: int
    seq: int
    key_valid: Optional[torch.Tensor] = None
    written: bool = False

    def _args(self, M: int):
        if self.workspace.dtype != torch.uint8 or self.workspace.dim() != 1:
            raise ValueError("the key-bound workspace is a 1-D uint8 tensor")
        kv = _mask_ptr(self.key_valid, (M // self.seq, self.seq)) if M % self.seq == 0 and \
            self.key_valid is not None else 0
        return (self.workspace.data_ptr(), self.k_col0, self.heads, self.head_dim, self.seq, kv)


def attention_workspace(B: int, S_q: int, S_k: int, H: int, head_dim: int, dtype: torch.dtype,
                        device: torch.device) -> torch.Tensor:
    """A workspace for ``attention(..., workspace=...)`` on ``[B, S, H, head_dim]`` problems of
    ``dtype``: the key-norm bounds and the redo flags (``mi355_attn_workspace_bytes_forced``);
    empty when the problem does not run on the matrix-core kernel."""
    n = _lib.lib().mi355_attn_workspace_bytes_forced(_lib.dtype_code(dtype), B, H, S_q, S_k,
                                                     head_dim)
    return torch.empty((max(int(n), 0),), device=device, dtype=torch.uint8)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _on_gpu(*tensors: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"expected a GPU tensor, got one on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    if dev is None:
        raise ValueError("no tensor given")
    return dev


def _mask_ptr(mask: Optional[torch.Tensor], shape: Tuple[int, ...]) -> int:
    if mask is None:
        return 0
    if mask.dtype not in (torch.bool, torch.uint8):
        raise TypeError("masks must be bool or uint8")
    if tuple(mask.shape) != tuple(shape) or not mask.is_contiguous():
        raise ValueError(f"mask must be a contiguous tensor of shape {shape}")
    return mask.data_ptr()


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
           out: Optional[torch.Tensor] = None, row_valid: Optional[torch.Tensor] = None,
           out_dtype: Optional[torch.dtype] = None,
           residual: Optional[torch.Tensor] = None, gelu: bool = False,
           zero_masked_rows: bool = False,
           key_bounds: Optional[KeyBoundTarget] = None) -> torch.Tensor:
    """``out[M, N] = x[M, K] @ weight[N, K]^T + bias[N]`` (nn.Linear), fp32 accumulate.

    ``x`` may be a row-strided 2-D view (unit column stride); ``weight`` must be contiguous and
    of x's dtype; ``bias`` is fp32. ``out_dtype`` (default x's dtype) may be any of fp32 /
    fp16 / bf16 for 16-bit inputs, and fp32 or fp16 for fp32 inputs. Rows whose ``row_valid`` entry is False are written as zeros.
    With ``residual`` ([M, N] of out_dtype, unit column stride; may be ``out`` itself) the result
    is ``residual + out_dtype(projection)``, masked rows giving ``residual`` -- or zeros with
    ``zero_masked_rows`` (the block's trailing masked_fill). ``gelu`` applies the exact GELU to
    the projection rounded to out_dtype (``F.gelu(nn.Linear(...)(x))``); it excludes
    ``residual`` and ``row_valid``. With ``key_bounds`` (a QKV projection; no residual, GELU
    or row mask) the epilogue also writes the attention's key-norm bounds when the shapes allow
    (``key_bounds.written``).
    """
    _on_gpu(x, weight, bias, out, row_valid, residual)
    if x.dim() != 2 or weight.dim() != 2:
        raise ValueError("linear expects 2-D x and weight")
    M, K = x.shape
    N, K2 = weight.shape
    if K2 != K:
        raise ValueError(f"inner sizes differ: x has K={K}, weight has K={K2}")
    dt = x.dtype
    odt = out_dtype or (out.dtype if out is not None else dt)
    if weight.dtype != dt:
        raise TypeError("x and weight must share one dtype")
    if x.stride(1) != 1 or not weight.is_contiguous():
        raise ValueError("x needs unit column stride and weight must be contiguous")
    if bias is not None and (bias.shape != (N,) or bias.dtype != torch.float32
                             or not bias.is_contiguous()):
        raise ValueError(f"bias must be a contiguous fp32 tensor of shape ({N},)")
    if out is None:
        out = torch.empty((M, N), device=x.device, dtype=odt)
    elif out.shape != (M, N) or out.dtype != odt or out.stride(1) != 1:
        raise ValueError("out must be [M, N] of out_dtype with unit column stride")
    if gelu:
        if residual is not None or row_valid is not None:
            raise ValueError("the GELU epilogue takes no residual or row mask")
        st = _lib.lib().mi355_gemm_bias_gelu(
            _lib.dtype_code(dt), _lib.dtype_code(odt), x.data_ptr(), x.stride(0),
            weight.data_ptr(), weight.stride(0), bias.data_ptr() if bias is not None else 0,
            out.data_ptr(), out.stride(0), M, N, K, _stream(x))
        _lib.check("mi355_gemm_bias_gelu", st)
        return out
    if zero_masked_rows and residual is None:
        raise ValueError("zero_masked_rows is a mode of the residual epilogue")
    if residual is not None:
        if residual.shape != (M, N) or residual.dtype != odt or residual.stride(1) != 1:
            raise ValueError("residual must be [M, N] of out_dtype with unit column stride")
        fn = "mi355_gemm_bias_residual_zero_masked" if zero_masked_rows else "mi355_gemm_bias_residual"
        st = getattr(_lib.lib(), fn)(
            _lib.dtype_code(dt), _lib.dtype_code(odt), x.data_ptr(), x.stride(0),
            weight.data_ptr(), weight.stride(0), bias.data_ptr() if bias is not None else 0,
            residual.data_ptr(), residual.stride(0), out.data_ptr(), out.stride(0), M, N, K,
            _mask_ptr(row_valid, (M,)), _stream(x))
        _lib.check(fn, st)
        return out
    if key_bounds is not None:
        if row_valid is not None:
            raise ValueError("the key-bound epilogue takes no row mask")
        _on_gpu(x, key_bounds.workspace, key_bounds.key_valid)
        st = _lib.lib().mi355_gemm_bias_kbound(
            _lib.dtype_code(dt), _lib.dtype_code(odt), x.data_ptr(), x.stride(0),
            weight.data_ptr(), weight.stride(0), bias.data_ptr() if bias is not None else 0,
            out.data_ptr(), out.stride(0), M, N, K, *key_bounds._args(M), _stream(x))
        key_bounds.written = st == 0
        if st != _E_UNSUPPORTED:
            _lib.check("mi355_gemm_bias_kbound", st)
            return out
    st = _lib.lib().mi355_gemm_bias(
        _lib.dtype_code(dt), _lib.dtype_code(odt), x.data_ptr(), x.stride(0), weight.data_ptr(),
        weight.stride(0), bias.data_ptr() if bias is not None else 0, out.data_ptr(),
        out.stride(0), M, N, K, _mask_ptr(row_valid, (M,)), _stream(x))
    _lib.check("mi355_gemm_bias", st)
    return out


def layer_norm(x: torch.Tensor, weight: Optional[torch.Tensor], bias: Optional[torch.Tensor],
               eps: float = 1e-5, out: Optional[torch.Tensor] = None,
               row_valid: Optional[torch.Tensor] = None,
               out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Row LayerNorm of a 2-D ``x`` (nn.LayerNorm over the last dimension): fp32 statistics,
    output rounded once to x's dtype, or to ``out_dtype`` (fp16 for an fp32 x: the fp16 operand
    of an fp32 model's projection). ``weight``/``bias`` are contiguous ``[K]`` of x's dtype.
    Rows whose ``row_valid`` entry is False are written as zeros."""
    _on_gpu(x, weight, bias, out, row_valid)
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("layer_norm expects a 2-D x with unit column stride")
    M, K = x.shape
    for t in (weight, bias):
        if t is not None and (t.shape != (K,) or t.dtype != x.dtype or not t.is_contiguous()):
            raise ValueError(f"LayerNorm weight/bias must be contiguous [{K}] of x's dtype")
    odt = out_dtype or (out.dtype if out is not None else x.dtype)
    if out is None:
        out = torch.empty((M, K), device=x.device, dtype=odt)
    elif out.shape != (M, K) or out.dtype != odt or out.stride(1) != 1:
        raise ValueError("out must be [M, K] of the output dtype with unit column stride")
    if odt != x.dtype:
        if row_valid is not None:
            raise ValueError("a converting LayerNorm takes no row mask")
        st = _lib.lib().mi355_layernorm_cvt(
            _lib.dtype_code(x.dtype), _lib.dtype_code(odt), x.data_ptr(), x.stride(0),
            weight.data_ptr() if weight is not None else 0,
            bias.data_ptr() if bias is not None else 0, float(eps), out.data_ptr(), out.stride(0),
            M, K, _stream(x))
        _lib.check("mi355_layernorm_cvt", st)
        return out
    if row_valid is not None:
        st = _lib.lib().mi355_layernorm_masked(
            _lib.dtype_code(x.dtype), x.data_ptr(), x.stride(0),
            weight.data_ptr() if weight is not None else 0,
            bias.data_ptr() if bias is not None else 0, float(eps), out.data_ptr(), out.stride(0),
            M, K, _mask_ptr(row_valid, (M,)), _stream(x))
        _lib.check("mi355_layernorm_masked", st)
        return out
    st = _lib.lib().mi355_layernorm(
        _lib.dtype_code(x.dtype), x.data_ptr(), x.stride(0),
        weight.data_ptr() if weight is not None else 0, bias.data_ptr() if bias is not None else 0,
        float(eps), out.data_ptr(), out.stride(0), M, K, _stream(x))
    _lib.check("mi355_layernorm", st)
    return out


def fold_layernorm(weight: torch.Tensor, bias: Optional[torch.Tensor],
                   gamma: Optional[torch.Tensor], beta: Optional[torch.Tensor],
                   dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Host-side fold of a LayerNorm (gamma, beta) into the projection that consumes it, for
    ``layernorm_linear``: returns ``(Wf [N, K] of dtype, colsum [N] fp32, bias' [N] fp32)`` with
    ``Wf = dtype(W * gamma)``, ``colsum = sum_k Wf[:, k]`` (of the rounded Wf, so the epilogue's
    mean subtraction cancels exactly against the weights the GEMM uses) and
    ``bias' = b + W @ beta``; the sums are formed in fp64. Run once per weight version."""
    with torch.no_grad():
        w64 = weight.detach().to(torch.float64)
        g = gamma.detach().to(torch.float64) if gamma is not None else None
        wf = (w64 * g[None, :] if g is not None else w64).to(dtype).contiguous()
        colsum = wf.to(torch.float64).sum(dim=1).to(torch.float32).contiguous()
        b = (bias.detach().to(torch.float64) if bias is not None
             else torch.zeros(weight.shape[0], dtype=torch.float64, device=weight.device))
        if beta is not None:
            b = b + w64 @ beta.detach().to(torch.float64)
        return wf, colsum, b.to(torch.float32).contiguous()


def layernorm_linear(x: torch.Tensor, weight: torch.Tensor, colsum: torch.Tensor,
                     bias: Optional[torch.Tensor], eps: float = 1e-5,
                     out_dtype: Optional[torch.dtype] = None, gelu: bool = False,
                     out: Optional[torch.Tensor] = None,
                     stats: Optional[torch.Tensor] = None,
                     key_bounds: Optional[KeyBoundTarget] = None) -> torch.Tensor:
    """``nn.Linear(nn.LayerNorm(x))`` (optionally followed by the exact GELU) without writing the
    normalised rows: ``weight``, ``colsum`` and ``bias`` come from ``fold_layernorm``. ``x`` is a
    2-D row-strided tensor (unit column stride); the row statistics go to ``stats`` ([M, 2] fp32
    workspace, allocated when not given). ``out_dtype`` defaults to x's dtype (a bf16 or fp32
    input may give fp16). ``key_bounds`` as for ``linear`` (not with ``gelu``)."""
    _on_gpu(x, weight, colsum, bias, out, stats)
    if x.dim() != 2 or weight.dim() != 2 or x.stride(1) != 1:
        raise ValueError("layernorm_linear expects a 2-D x with unit column stride and 2-D weight")
    M, K = x.shape
    N, K2 = weight.shape
    if K2 != K:
        raise ValueError(f"inner sizes differ: x has K={K}, weight has K={K2}")
    if weight.dtype != x.dtype or not weight.is_contiguous():
        raise ValueError("weight must be contiguous and of x's dtype")
    if colsum.shape != (N,) or colsum.dtype != torch.float32 or not colsum.is_contiguous():
        raise ValueError(f"colsum must be a contiguous fp32 tensor of shape ({N},)")
    if bias is not None and (bias.shape != (N,) or bias.dtype != torch.float32
                             or not bias.is_contiguous()):
        raise ValueError(f"bias must be a contiguous fp32 tensor of shape ({N},)")
    odt = out_dtype or (out.dtype if out is not None else x.dtype)
    if out is None:
        out = torch.empty((M, N), device=x.device, dtype=odt)
    elif out.shape != (M, N) or out.dtype != odt or out.stride(1) != 1:
        raise ValueError("out must be [M, N] of out_dtype with unit column stride")
    if stats is None:
        stats = torch.empty((M, 2), device=x.device, dtype=torch.float32)
    elif stats.shape != (M, 2) or stats.dtype != torch.float32 or not stats.is_contiguous():
        raise ValueError(f"stats must be a contiguous fp32 tensor of shape ({M}, 2)")
    if key_bounds is not None:
        if gelu:
            raise ValueError("the key-bound epilogue takes no GELU")
        _on_gpu(x, key_bounds.workspace, key_bounds.key_valid)
        st = _lib.lib().mi355_layernorm_gemm_bias_kbound(
            _lib.dtype_code(x.dtype), _lib.dtype_code(odt), x.data_ptr(), x.stride(0),
            weight.data_ptr(), weight.stride(0), colsum.data_ptr(),
            bias.data_ptr() if bias is not None else 0, float(eps), stats.data_ptr(),
            out.data_ptr(), out.stride(0), M, N, K, *key_bounds._args(M), _stream(x))
        key_bounds.written = st == 0
        if st != _E_UNSUPPORTED:
            _lib.check("mi355_layernorm_gemm_bias_kbound", st)
            return out
    st = _lib.lib().mi355_layernorm_gemm_bias(
        _lib.dtype_code(x.dtype), _lib.dtype_code(odt), x.data_ptr(), x.stride(0),
        weight.data_ptr(), weight.stride(0), colsum.data_ptr(),
        bias.data_ptr() if bias is not None else 0, float(eps), stats.data_ptr(), out.data_ptr(),
        out.stride(0), M, N, K, _lib.EPI_GELU if gelu else 0, _stream(x))
    _lib.check("mi355_layernorm_gemm_bias", st)
    return out


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: Optional[torch.Tensor] = None,
              scale: Optional[float] = None, causal: bool = False,
              key_valid: Optional[torch.Tensor] = None,
              key_bound: Optional[bool] = None,
              workspace: Optional[torch.Tensor] = None, bounds_ready: bool = False,
              causal_sweep_min_keys: Optional[int] = None) -> torch.Tensor:
    """Streamed softmax attention over ``[B, S, H, head_dim]`` views (unit head_dim stride).

    ``out`` defaults to a new contiguous ``[B, S_q, H, head_dim]`` tensor, whose
    ``view(B, S_q, H * head_dim)`` is the merged-head context of the reference block.
    ``key_valid`` is an optional ``[B, S_k]`` bool mask of keys to attend to.
    ``key_bound`` selects the key-norm bound pass of the matrix-core kernel (a workspace of
    per-chunk max |k| that lets waves skip the per-tile row maxima, and of the offset sweep's
    redo flags): None = the library's choice (``mi355_attn_workspace_bytes``: long key
    ranges), True = always (``mi355_attn_workspace_bytes_forced``), False = never. With the
    workspace, a key mask is resolved on the device: work-groups whose keys are all valid run
    the unmasked sweeps, the others a second, key-masked launch; nothing synchronises the host.
    ``workspace`` (``attention_workspace``) supplies the workspace instead, with
    ``bounds_ready`` when a QKV projection already wrote the bounds into it
    (``KeyBoundTarget``) and ``causal_sweep_min_keys`` the key range from which causal query
    tiles take the sweeps (``mi355_attn_fwd_kb``; default 32768, the library's choice).
    """
    _on_gpu(q, k, v, out, key_valid)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 4-D [B, S, H, head_dim] views")
    B, Sq, H, D = q.shape
    Bk, Sk, Hk, Dk = k.shape
    if (Bk, Hk, Dk) != (B, H, D) or tuple(v.shape) != (B, Sk, H, D):
        raise ValueError(f"shape mismatch q={tuple(q.shape)} k={tuple(k.shape)} v={tuple(v.shape)}")
    dt = q.dtype
    if k.dtype != dt or v.dtype != dt:
        raise TypeError("q, k, v must share one dtype")
    if q.stride(3) != 1 or k.stride(3) != 1 or v.stride(3) != 1:
        raise ValueError("head_dim must be the unit-stride dimension")
    if out is None:
        out = torch.empty((B, Sq, H, D), device=q.device, dtype=dt)
    elif tuple(out.shape) != (B, Sq, H, D) or out.dtype != dt or out.stride(3) != 1:
        raise ValueError("out must be [B, S_q, H, head_dim] of q's dtype with unit head_dim stride")
    if scale is None:
        scale = D ** -0.5
    kv_ptr, kv_sb = 0, 0
    if key_valid is not None:
        kv_ptr = _mask_ptr(key_valid, (B, Sk))
        kv_sb = key_valid.stride(0)
    L = _lib
    code = L.dtype_code(dt)
    if workspace is not None or bounds_ready or causal_sweep_min_keys is not None:
        if workspace is None:
            raise ValueError("bounds_ready / causal_sweep_min_keys need a workspace")
        _on_gpu(q, workspace)
        if workspace.dtype != torch.uint8 or workspace.dim() != 1:
            raise ValueError("workspace must be a 1-D uint8 tensor")
        need = L.lib().mi355_attn_workspace_bytes_forced(code, B, H, Sq, Sk, D)
        if workspace.numel() < need:
            raise ValueError(f"workspace holds {workspace.numel()} bytes, {need} needed")
        gate = 32768 if causal_sweep_min_keys is None else int(causal_sweep_min_keys)
        st = L.lib().mi355_attn_fwd_kb(
            code, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, H, Sq, Sk, D,
            L.i64_array((q.stride(0), q.stride(1), q.stride(2))),
            L.i64_array((k.stride(0), k.stride(1), k.stride(2))),
            L.i64_array((v.stride(0), v.stride(1), v.stride(2))),
            L.i64_array((out.stride(0), out.stride(1), out.stride(2))),
            float(scale), 1 if causal else 0, kv_ptr, kv_sb,
            workspace.data_ptr() if need > 0 else 0, workspace.numel() if need > 0 else 0,
            1 if (bounds_ready and need > 0) else 0, gate, _stream(q))
        L.check("mi355_attn_fwd_kb", st)
        return out
    if key_bound is None:
        ws_bytes = L.lib().mi355_attn_workspace_bytes(code, B, H, Sq, Sk, D)
    elif key_bound:
        ws_bytes = L.lib().mi355_attn_workspace_bytes_forced(code, B, H, Sq, Sk, D)
    else:
        ws_bytes = 0
    args = (code, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, H, Sq, Sk, D,
            L.i64_array((q.stride(0), q.stride(1), q.stride(2))),
            L.i64_array((k.stride(0), k.stride(1), k.stride(2))),
            L.i64_array((v.stride(0), v.stride(1), v.stride(2))),
            L.i64_array((out.stride(0), out.stride(1), out.stride(2))),
            float(scale), 1 if causal else 0, kv_ptr, kv_sb)
    if ws_bytes > 0:
        ws = torch.empty((ws_bytes,), device=q.device, dtype=torch.uint8)
        st = L.lib().mi355_attn_fwd_ws(*args, ws.data_ptr(), ws_bytes, _stream(q))
        L.check("mi355_attn_fwd_ws", st)
    else:
        st = L.lib().mi355_attn_fwd(*args, _stream(q))
        L.check("mi355_attn_fwd", st)
    return out


def quant_rows_i8(x: torch.Tensor, mode: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-row symmetric int8 quantisation; returns ``(q [M, K] int8, scale [M] fp32)``.

    mode 0 is the activation recipe (scale = max(amax, 1e-6) / 127), mode 1 the weight recipe
    (scale = max(amax / 127, 1e-8)).
    """
    _on_gpu(x)
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("quant_rows_i8 expects a 2-D tensor with unit column stride")
    M, K = x.shape
    q = torch.empty((M, K), device=x.device, dtype=torch.int8)
    s = torch.empty((M,), device=x.device, dtype=torch.float32)
    st = _lib.lib().mi355_quant_rows_i8(_lib.dtype_code(x.dtype), x.data_ptr(), x.stride(0),
                                        q.data_ptr(), s.data_ptr(), M, K, int(mode), _stream(x))
    _lib.check("mi355_quant_rows_i8", st)
    return q, s


def linear_i8(a: torch.Tensor, w: torch.Tensor, s_a: torch.Tensor, s_w: torch.Tensor,
              bias: Optional[torch.Tensor] = None, out_dtype: torch.dtype = torch.float16,
              out: Optional[torch.Tensor] = None, acc_out: Optional[torch.Tensor] = None,
              row_valid: Optional[torch.Tensor] = None, want_out: bool = True,
              residual: Optional[torch.Tensor] = None, gelu: bool = False,
              zero_masked_rows: bool = False) -> Optional[torch.Tensor]:
    """W8A8 projection: ``y = fp32(a @ w^T) * (s_a[:, None] * s_w[None, :]) + bias``.

    ``a`` is ``[M, K]`` int8, ``w`` is ``[N, K]`` int8 (K-major), scales fp32. ``acc_out``
    (``[M, N]`` int32) receives the raw int32 accumulators when given. Epilogues of the int8
    transformer block (k008_int8_gemm.py:221-233), each computed in fp32 from y rounded to
    ``out_dtype`` and rounded once: ``gelu`` gives gelu(y); ``residual`` ([M, N] of out_dtype,
    may be ``out``) gives residual + y with masked rows keeping the residual, or zeroed with
    ``zero_masked_rows``. The epilogues do not combine with ``acc_out``.
    """
    _on_gpu(a, w, s_a, s_w, bias, out, acc_out, row_valid, residual)
    if a.dtype != torch.int8 or w.dtype != torch.int8:
        raise TypeError("a and w must be int8")
    if not a.is_contiguous() or not w.is_contiguous():
        raise ValueError("a and w must be contiguous")
    M, K = a.shape
    N, K2 = w.shape
    if K2 != K:
        raise ValueError("inner sizes differ")
    if s_a.shape != (M,) or s_w.shape != (N,) or s_a.dtype != torch.float32 or s_w.dtype != torch.float32:
        raise ValueError("s_a [M] and s_w [N] must be fp32")
    if bias is not None and (bias.shape != (N,) or bias.dtype != torch.float32):
        raise ValueError("bias must be fp32 [N]")
    if acc_out is not None and (acc_out.shape != (M, N) or acc_out.dtype != torch.int32
                                or not acc_out.is_contiguous()):
        raise ValueError("acc_out must be a contiguous int32 [M, N] tensor")
    epilogue = gelu or residual is not None or zero_masked_rows
    if epilogue and acc_out is not None:
        raise ValueError("acc_out does not combine with the gelu / residual epilogues")
    if zero_masked_rows and residual is None:
        raise ValueError("zero_masked_rows needs a residual")
    if gelu and residual is not None:
        raise ValueError("gelu does not combine with a residual")
    if residual is not None and (residual.shape != (M, N) or residual.dtype != out_dtype
                                 or residual.stride(1) != 1):
        raise ValueError("residual must be [M, N] of out_dtype with unit column stride")
    if (want_out or epilogue) and out is None:
        out = torch.empty((M, N), device=a.device, dtype=out_dtype)
    if out is not None and (out.shape != (M, N) or out.dtype != out_dtype or out.stride(1) != 1):
        raise ValueError("out must be [M, N] of out_dtype with unit column stride")
    mask = _mask_ptr(row_valid, (M,))
    if epilogue:
        flags = (_lib.EPI_GELU if gelu else 0) | (_lib.EPI_ZERO_MASKED if zero_masked_rows else 0)
        st = _lib.lib().mi355_gemm_i8_epilogue(
            a.data_ptr(), w.data_ptr(), s_a.data_ptr(), s_w.data_ptr(),
            bias.data_ptr() if bias is not None else 0, _lib.dtype_code(out_dtype),
            out.data_ptr(), out.stride(0),
            residual.data_ptr() if residual is not None else 0,
            residual.stride(0) if residual is not None else N, M, N, K, mask, flags, _stream(a))
        _lib.check("mi355_gemm_i8_epilogue", st)
        return out
    st = _lib.lib().mi355_gemm_i8(
        a.data_ptr(), w.data_ptr(), s_a.data_ptr(), s_w.data_ptr(),
        bias.data_ptr() if bias is not None else 0, _lib.dtype_code(out_dtype),
        out.data_ptr() if out is not None else 0, out.stride(0) if out is not None else N,
        acc_out.data_ptr() if acc_out is not None else 0, M, N, K,
        mask, _stream(a))
    _lib.check("mi355_gemm_i8", st)
    return out
