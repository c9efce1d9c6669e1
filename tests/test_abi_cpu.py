"""C-ABI checks that need no GPU: the library loads, exports every symbol the header declares,
and rejects invalid arguments with its documented negative status codes before touching the
device (every call below fails argument validation, so no kernel is launched)."""
import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mi355attn.h"


def _lib():
    from tiktok_techjam_2026_track3_amd import _lib
    return _lib


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mi355_\w+)\s*\(", text)))


def _status_codes():
    return {m.group(1): int(m.group(2))
            for m in re.finditer(r"#define\s+(MI355_\w+)\s+\(?(-?\d+)\)?", HEADER.read_text())}


def test_library_exports_every_declared_symbol():
    L = _lib()
    h = L.lib()
    declared = _declared_functions()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(h, name), f"{name} declared in {HEADER.name} but not exported"
    assert set(declared) == set(L.EXPORTED), "ctypes signature table out of sync with the header"


def test_version_and_status_strings():
    L = _lib()
    assert L.lib().mi355_version() >= 100
    codes = _status_codes()
    for name, code in codes.items():
        if name.startswith("MI355_E_"):
            msg = L.status_string(code)
            assert msg and msg != "unknown status", name


def test_dtype_codes_match_header():
    import torch
    L = _lib()
    codes = _status_codes()
    assert L.dtype_code(torch.float32) == codes["MI355_F32"]
    assert L.dtype_code(torch.float16) == codes["MI355_F16"]
    assert L.dtype_code(torch.bfloat16) == codes["MI355_BF16"]
    with pytest.raises(TypeError):
        L.dtype_code(torch.int32)


def test_gemm_argument_validation():
    L = _lib()
    h = L.lib()
    codes = _status_codes()
    fake = 1 << 20                                   # aligned, never dereferenced
    assert h.mi355_gemm_bias(1, 1, fake, 64, fake, 64, None, fake, 64, -1, 64, 64, None, None) == codes["MI355_E_BAD_SIZE"]
    assert h.mi355_gemm_bias(1, 1, None, 64, fake, 64, None, fake, 64, 4, 64, 64, None, None) == codes["MI355_E_NULL_POINTER"]
    assert h.mi355_gemm_bias(7, 1, fake, 64, fake, 64, None, fake, 64, 4, 64, 64, None, None) == codes["MI355_E_BAD_DTYPE"]
    assert h.mi355_gemm_bias(1, 1, fake, 64, fake, 64, None, fake, 64, 4, 64, 60, None, None) == codes["MI355_E_ALIGNMENT"]
    assert h.mi355_gemm_bias(1, 1, fake + 2, 64, fake, 64, None, fake, 64, 4, 64, 64, None, None) == codes["MI355_E_ALIGNMENT"]
    # fp32 inputs give fp32 or fp16 (an fp32 model's fp16 attention core), never bf16
    assert h.mi355_gemm_bias(0, 2, fake, 64, fake, 64, None, fake, 64, 4, 64, 64, None, None) == codes["MI355_E_UNSUPPORTED"]
    assert h.mi355_gemm_bias(1, 1, fake, 32, fake, 64, None, fake, 64, 4, 64, 64, None, None) == codes["MI355_E_BAD_SIZE"]
    # empty problems are a successful no-op
    assert h.mi355_gemm_bias(1, 1, None, 64, None, 64, None, None, 64, 0, 64, 64, None, None) == 0


def test_residual_gemm_and_layernorm_argument_validation():
    L = _lib()
    h = L.lib()
    codes = _status_codes()
    fake = 1 << 20
    # residual GEMM: the residual pointer is required, its stride checked like the output's
    assert h.mi355_gemm_bias_residual(1, 1, fake, 64, fake, 64, None, None, 64, fake, 64, 4, 64, 64,
                                      None, None) == codes["MI355_E_NULL_POINTER"]
    assert h.mi355_gemm_bias_residual(1, 1, fake, 64, fake, 64, None, fake, 32, fake, 64, 4, 64, 64,
                                      None, None) == codes["MI355_E_BAD_SIZE"]
    assert h.mi355_gemm_bias_residual(1, 2, fake, 64, fake, 64, None, fake, 64, fake, 64, 0, 64, 64,
                                      None, None) == 0
    # LayerNorm: sizes, dtype, alignment and the one-wave row limit
    ln = h.mi355_layernorm
    assert ln(1, fake, 64, None, None, 1e-5, fake, 64, -1, 64, None) == codes["MI355_E_BAD_SIZE"]
    assert ln(1, fake, 64, None, None, 1e-5, fake, 64, 4, 0, None) == codes["MI355_E_BAD_SIZE"]
    assert ln(1, None, 64, None, None, 1e-5, fake, 64, 4, 64, None) == codes["MI355_E_NULL_POINTER"]
    assert ln(6, fake, 64, None, None, 1e-5, fake, 64, 4, 64, None) == codes["MI355_E_BAD_DTYPE"]
    assert ln(1, fake, 64, None, None, 1e-5, fake, 64, 4, 60, None) == codes["MI355_E_ALIGNMENT"]
    assert ln(1, fake, 64, fake + 2, None, 1e-5, fake, 64, 4, 64, None) == codes["MI355_E_ALIGNMENT"]
    assert ln(1, fake, 32, None, None, 1e-5, fake, 64, 4, 64, None) == codes["MI355_E_BAD_SIZE"]
    assert ln(1, fake, 64, None, None, -1.0, fake, 64, 4, 64, None) == codes["MI355_E_BAD_SIZE"]
    assert ln(1, fake, 16384, None, None, 1e-5, fake, 16384, 4, 16384, None) == codes["MI355_E_UNSUPPORTED"]
    assert ln(0, fake, 8192, None, None, 1e-5, fake, 8192, 4, 8192, None) == codes["MI355_E_UNSUPPORTED"]
    assert ln(1, fake, 64, None, None, 1e-5, fake, 64, 0, 64, None) == 0


def test_attention_argument_validation():
    L = _lib()
    h = L.lib()
    codes = _status_codes()
    fake = 1 << 20
    st = L.i64_array((3 * 64 * 4 * 16, 3 * 64 * 4, 64))
    ost = L.i64_array((64 * 4 * 16, 64 * 4, 64))

    def call(dtype=1, hd=64, B=2, S=16, q=fake, scale=0.125, strides=st):
        return h.mi355_attn_fwd(dtype, q, fake, fake, fake, B, 4, S, S, hd, strides, strides,
                                strides, ost, scale, 0, None, 0, None)

    assert call(hd=40) == codes["MI355_E_HEAD_DIM"]
    assert call(hd=512) == codes["MI355_E_HEAD_DIM"]
    assert call(hd=4) == codes["MI355_E_HEAD_DIM"]
    assert call(dtype=5) == codes["MI355_E_BAD_DTYPE"]
    assert call(q=None) == codes["MI355_E_NULL_POINTER"]
    assert call(q=fake + 8) == codes["MI355_E_ALIGNMENT"]
    assert call(scale=0.0) == codes["MI355_E_UNSUPPORTED"]
    assert call(B=-1) == codes["MI355_E_BAD_SIZE"]
    assert call(strides=L.i64_array((3, 64, 64))) == codes["MI355_E_ALIGNMENT"]
    assert call(B=0) == 0


def test_attention_workspace_argument_validation():
    """mi355_attn_fwd_ws: the recommended size is the key-norm bound array of the matrix-core
    kernel (B * H * ceil(S_k / 256) floats), rounded up to 256 bytes, then one int per
    work-group of 256 queries (the offset sweep's redo flags), from S_k = 32768 on, 0
    elsewhere (mi355_attn_workspace_bytes_forced: the same size at any key length); a non-NULL
    workspace below the bound size or misaligned is refused before any launch."""
    L = _lib()
    h = L.lib()
    codes = _status_codes()
    fake = 1 << 20
    B, H = 2, 4

    def size(S_q, S_k):
        return (B * H * -(-S_k // 256) * 4 + 255) // 256 * 256 + B * H * -(-S_q // 256) * 4
    assert h.mi355_attn_workspace_bytes(1, B, H, 32768, 32768, 64) == size(32768, 32768) == 8192
    assert h.mi355_attn_workspace_bytes(2, B, H, 10, 100000, 128) == size(10, 100000) == 12576
    assert h.mi355_attn_workspace_bytes(1, B, H, 40000, 40000, 32) == size(40000, 40000) == 10144
    assert h.mi355_attn_workspace_bytes(1, B, H, 8192, 8192, 64) == 0      # short key range
    assert h.mi355_attn_workspace_bytes(0, B, H, 8192, 8192, 64) == 0      # fp32: VALU kernel
    assert h.mi355_attn_workspace_bytes(1, B, H, 8192, 8192, 80) == 0      # head_dim 80: VALU
    # the forced size: the same layout at any key length, 0 off the matrix-core kernel
    assert h.mi355_attn_workspace_bytes_forced(1, B, H, 8192, 8192, 64) == size(8192, 8192) == 2048
    assert h.mi355_attn_workspace_bytes_forced(1, B, H, 100, 300, 128) == size(100, 300) == 288
    assert h.mi355_attn_workspace_bytes_forced(0, B, H, 8192, 8192, 64) == 0
    assert h.mi355_attn_workspace_bytes_forced(1, B, H, 8192, 8192, 80) == 0
    assert h.mi355_attn_workspace_bytes_forced(1, B, H, 8192, 0, 64) == 0
    S = 3000  # 12 chunks
    st = L.i64_array((3 * 64 * H * S, 3 * 64 * H, 64))
    ost = L.i64_array((64 * H * S, 64 * H, 64))

    def call(ws, nbytes):
        return h.mi355_attn_fwd_ws(1, fake, fake, fake, fake, B, H, S, S, 64, st, st, st, ost,
                                   0.125, 0, None, 0, ws, nbytes, None)

    need = B * H * 12 * 4
    assert call(fake, need - 4) == codes["MI355_E_BAD_SIZE"]
    assert call(fake + 2, need) == codes["MI355_E_ALIGNMENT"]
    # argument validation still precedes the workspace check
    assert h.mi355_attn_fwd_ws(1, fake, fake, fake, fake, B, H, S, S, 40, st, st, st, ost, 0.125, 0,
                               None, 0, fake, need, None) == codes["MI355_E_HEAD_DIM"]


def test_int8_argument_validation():
    L = _lib()
    h = L.lib()
    codes = _status_codes()
    fake = 1 << 20
    assert h.mi355_quant_rows_i8(1, fake, 64, fake, fake, 4, 60, 0, None) == codes["MI355_E_ALIGNMENT"]
    assert h.mi355_quant_rows_i8(1, fake, 64, fake, fake, 4, 64, 2, None) == codes["MI355_E_UNSUPPORTED"]
    assert h.mi355_quant_rows_i8(1, None, 64, fake, fake, 4, 64, 0, None) == codes["MI355_E_NULL_POINTER"]
    assert h.mi355_gemm_i8(fake, fake, fake, fake, None, 1, fake, 64, None, 4, 64, 40, None, None) == codes["MI355_E_ALIGNMENT"]
    assert h.mi355_gemm_i8(fake, fake, None, fake, None, 1, fake, 64, None, 4, 64, 64, None, None) == codes["MI355_E_NULL_POINTER"]
    assert h.mi355_gemm_i8(fake, fake, fake, fake, None, 9, fake, 64, None, 4, 64, 64, None, None) == codes["MI355_E_BAD_DTYPE"]
    # the epilogue variant: A, W, s_a, s_w, bias, out_dtype, C, ldc, R, ldr, M, N, K, row_valid,
    # epi, stream (every rejected call returns before any launch)
    ep = h.mi355_gemm_i8_epilogue
    gelu, zero = L.EPI_GELU, L.EPI_ZERO_MASKED
    assert ep(fake, fake, fake, fake, None, 1, fake, 64, None, 64, 4, 64, 40, None, gelu, None) == codes["MI355_E_ALIGNMENT"]
    assert ep(fake, fake, fake, fake, None, 1, fake, 64, fake, 64, 4, 64, 64, None, gelu, None) == codes["MI355_E_UNSUPPORTED"]
    assert ep(fake, fake, fake, fake, None, 1, fake, 64, None, 64, 4, 64, 64, None, 4, None) == codes["MI355_E_UNSUPPORTED"]
    assert ep(fake, fake, fake, None, None, 1, fake, 64, fake, 64, 4, 64, 64, None, zero, None) == codes["MI355_E_NULL_POINTER"]
    assert ep(fake, fake, fake, fake, None, 1, None, 64, fake, 64, 4, 64, 64, None, 0, None) == codes["MI355_E_NULL_POINTER"]
    assert ep(fake, fake, fake, fake, None, 9, fake, 64, fake, 64, 4, 64, 64, None, 0, None) == codes["MI355_E_BAD_DTYPE"]
    assert ep(fake, fake, fake, fake, None, 1, fake, 64, fake, 32, 4, 64, 64, None, zero, None) == codes["MI355_E_BAD_SIZE"]
    assert ep(fake, fake, fake, fake, None, 1, fake, 32, None, 64, 4, 64, 64, None, gelu, None) == codes["MI355_E_BAD_SIZE"]
    assert ep(fake, fake, fake, fake, None, 1, fake, 64, None, 64, 0, 64, 64, None, gelu, None) == 0


def test_kernel_error_carries_status():
    L = _lib()
    with pytest.raises(L.KernelError) as ei:
        L.check("mi355_attn_fwd", -5)
    assert ei.value.status == -5 and "head_dim" in str(ei.value)


def test_build_refuses_lds_dma_kernels_that_use_scratch():
    """build.py parses the compiler's kernel-resource-usage remarks and refuses an LDS-DMA kernel
    (attention MFMA / projection GEMM) that uses scratch memory or spills VGPRs."""
    import importlib
    B = importlib.import_module("tiktok_techjam_2026_track3_amd.build")
    remarks = "\n".join([
        "a.hip:1:1: remark: Function Name: _ZN12_GLOBAL__N_113attn_fwd_mfmaIDF16_Li64EEEvNS_8AttnArgsE [-R]",
        "a.hip:1:1: remark:     ScratchSize [bytes/lane]: 16 [-R]",
        "a.hip:1:1: remark:     SGPRs Spill: 0 [-R]",
        "a.hip:1:1: remark:     VGPRs Spill: 4 [-R]",
        "a.hip:2:1: remark: Function Name: _ZN12_GLOBAL__N_113attn_fwd_valuIfLi8EEEvNS_8AttnArgsE [-R]",
        "a.hip:2:1: remark:     ScratchSize [bytes/lane]: 8 [-R]",
        "a.hip:2:1: remark:     VGPRs Spill: 2 [-R]",
    ])
    usage = B.resource_usage(remarks)
    assert usage["_ZN12_GLOBAL__N_113attn_fwd_mfmaIDF16_Li64EEEvNS_8AttnArgsE"] == {
        "scratch": 16, "sgpr_spill": 0, "vgpr_spill": 4}
    with pytest.raises(RuntimeError, match="must not use scratch"):
        B.check_no_scratch("a.hip", usage)
    # the vector-ALU kernel issues no LDS-DMA loads: not checked
    B.check_no_scratch("a.hip", {k: v for k, v in usage.items() if "valu" in k})


def test_layernorm_cvt_argument_validation():
    """mi355_layernorm_cvt: same-dtype calls are mi355_layernorm; fp32 -> fp16 is the one
    converting pair; the checks run before any launch."""
    L = _lib()
    h = L.lib()
    codes = _status_codes()
    fake = 1 << 20
    cvt = h.mi355_layernorm_cvt
    assert cvt(0, 2, fake, 64, None, None, 1e-5, fake, 64, 4, 64, None) == codes["MI355_E_UNSUPPORTED"]
    assert cvt(1, 0, fake, 64, None, None, 1e-5, fake, 64, 4, 64, None) == codes["MI355_E_UNSUPPORTED"]
    assert cvt(0, 7, fake, 64, None, None, 1e-5, fake, 64, 4, 64, None) == codes["MI355_E_BAD_DTYPE"]
    assert cvt(0, 1, fake, 64, None, None, 1e-5, fake, 64, 4, 62, None) == codes["MI355_E_ALIGNMENT"]
    assert cvt(0, 1, fake, 64, None, None, 1e-5, fake + 4, 64, 4, 64, None) == codes["MI355_E_ALIGNMENT"]
    assert cvt(0, 1, None, 64, None, None, 1e-5, fake, 64, 4, 64, None) == codes["MI355_E_NULL_POINTER"]
    assert cvt(0, 1, fake, 64, None, None, -1.0, fake, 64, 4, 64, None) == codes["MI355_E_BAD_SIZE"]
    assert cvt(0, 1, fake, 32, None, None, 1e-5, fake, 64, 4, 64, None) == codes["MI355_E_BAD_SIZE"]
    assert cvt(0, 1, fake, 8192, None, None, 1e-5, fake, 8192, 4, 8192, None) == codes["MI355_E_UNSUPPORTED"]
    assert cvt(0, 1, fake, 64, None, None, 1e-5, fake, 64, 0, 64, None) == 0


def test_noalloc_rejects_rows_beyond_the_array():
    """mi355_layernorm_gemm_bias_noalloc checks M against its file-scope array (2^20 rows,
    MI355_NOALLOC_MAX_ROWS) on the host, before any device call: with aligned pointers that are
    never dereferenced, M = 2^20 + 1 is the size error and nothing is launched."""
    L = _lib()
    h = L.lib()
    codes = _status_codes()
    fake = 1 << 20                                   # aligned, never dereferenced
    rc = h.mi355_layernorm_gemm_bias_noalloc(1, 1, fake, 64, fake, 64, fake, fake, 1e-5, fake, 32,
                                             (1 << 20) + 1, 32, 64, 0, None)
    assert rc == codes["MI355_E_BAD_SIZE"]


def test_key_bound_entry_points_argument_validation():
    """mi355_gemm_bias_kbound / mi355_layernorm_gemm_bias_kbound refuse, before any launch,
    what their epilogue cannot serve (MI355_E_UNSUPPORTED: the caller then runs the plain
    projection and the attention's bound pass) and malformed bound arguments; mi355_attn_fwd_kb
    needs a workspace for ready bounds and a non-negative causal sweep length."""
    L = _lib()
    h = L.lib()
    codes = _status_codes()
    fake = 1 << 20
    F16, BF16, F32 = 1, 2, 0
    B, S, d, H, hd = 2, 768, 512, 8, 64
    M, N, K = B * S, 3 * d, d

    def gemm(in_dt=F16, out_dt=F16, kb=fake, col0=d, heads=H, head_dim=hd, seq=S, ldc=N, m=M):
        return h.mi355_gemm_bias_kbound(in_dt, out_dt, fake, K, fake, K, fake, fake, ldc, m, N, K,
                                        kb, col0, heads, head_dim, seq, None, None)

    assert gemm(kb=None) == codes["MI355_E_NULL_POINTER"]
    assert gemm(kb=fake + 2) == codes["MI355_E_ALIGNMENT"]
    assert gemm(head_dim=80) == codes["MI355_E_HEAD_DIM"]
    assert gemm(m=M - 256) == codes["MI355_E_BAD_SIZE"]          # rows not whole sequences
    assert gemm(col0=2 * d + 256) == codes["MI355_E_BAD_SIZE"]   # K block past the columns
    assert gemm(seq=700, m=2 * 700) == codes["MI355_E_UNSUPPORTED"]   # chunks straddle tiles
    assert gemm(col0=384, heads=6) == codes["MI355_E_UNSUPPORTED"]    # K block not on a tile
    assert gemm(out_dt=F32) == codes["MI355_E_UNSUPPORTED"]
    assert gemm(in_dt=F32) == codes["MI355_E_UNSUPPORTED"]           # fp32 operands
    assert gemm(ldc=N + 4) == codes["MI355_E_UNSUPPORTED"]           # rows not 16-byte aligned
    assert gemm(m=256, seq=256) == codes["MI355_E_UNSUPPORTED"]      # split-K sized problem
    assert h.mi355_layernorm_gemm_bias_kbound(BF16, F16, fake, K, fake, K, fake, fake, 1e-5, fake,
                                              fake, N, M, N, K, fake, d, H, hd, 700, None,
                                              None) == codes["MI355_E_BAD_SIZE"]
    assert h.mi355_layernorm_gemm_bias_kbound(F32, F16, fake, K, fake, K, fake, fake, 1e-5, fake,
                                              fake, N, M, N, K, fake, d, H, hd, S, None,
                                              None) == codes["MI355_E_UNSUPPORTED"]
    st = L.i64_array((3 * d * S, 3 * d, hd))
    ost = L.i64_array((d * S, d, hd))

    def attn(ws, nbytes, ready, gate):
        return h.mi355_attn_fwd_kb(F16, fake, fake, fake, fake, B, H, S, S, hd, st, st, st, ost,
                                   0.125, 1, None, 0, ws, nbytes, ready, gate, None)

    assert attn(None, 0, 1, 2048) == codes["MI355_E_NULL_POINTER"]
    assert attn(fake, 1 << 16, 0, -1) == codes["MI355_E_BAD_SIZE"]
    assert attn(fake, 4, 1, 2048) == codes["MI355_E_BAD_SIZE"]       # smaller than the bounds
