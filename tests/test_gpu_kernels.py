"""GPU parity of each kernel against the CPU oracle, through the C-ABI (ops wrappers).

Floating-point kernels are checked against an fp64 evaluation of the same (already rounded)
inputs with an explicit error bound built from the rounding points of the kernel:
  GEMM:      |out - ref| <= u_out*|ref| + 4*K*2^-24 * (|A|·|W|^T) + 1e-7
  attention: |out - ref| <= (2*u_p + 2^-18 + 2^-22*L + 2 ln2 u_in c max_j |q_i|.|k_j|) * (P·|V|)
                             + u_out*|ref| + 1e-7
where u = 2^-11 (fp16), 2^-8 (bf16), 2^-24 (fp32) is the unit round-off of the type the value is
rounded to (probabilities P for u_p, the stored output for u_out), L = max|s*scale*log2(e)|
(the exp2 argument's fp32 rounding) and c = scale*log2(e) (the kernel re-rounds c*q). The int8 kernels are compared bit for bit.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import int8 as OI

pytestmark = pytest.mark.gpu

UNIT = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8, torch.float32: 2.0 ** -24}


def _ops():
    from tiktok_techjam_2026_track3_amd import ops
    return ops


def _rand(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _report(name, err, bound):
    worst = float((err / bound).max())
    print(f"{name}: max_err={float(err.max()):.3g} worst err/bound={worst:.3f}", flush=True)
    return worst


# --------------------------------------------------------------------------------- GEMM
GEMM_SHAPES = [(1, 64, 64), (128, 768, 256), (300, 200, 136), (513, 130, 1024), (2048, 3072, 1024),
               (1000, 1536, 512), (4096, 4096, 64), (65536, 128, 128)]


@pytest.mark.parametrize("dtype,out_dtype", [(torch.float16, torch.float16),
                                             (torch.bfloat16, torch.bfloat16),
                                             (torch.float32, torch.float32),
                                             (torch.bfloat16, torch.float16),
                                             (torch.float16, torch.bfloat16),
                                             (torch.float32, torch.float16),
                                             (torch.float16, torch.float32),
                                             (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_linear_error_bound(gpu, dtype, out_dtype, M, N, K):
    """Every operand / output type pair, on shapes that take the split-K kernel (at most 512
    tiles of 32 x 32: the first four), the tiled kernel at each of its 16-bit tile sizes
    (128 x 128 for 2048 x 3072 and for 65536 x 128, 64 x 64 for 1000 x 1536, 256 x 256 for
    4096 x 4096 x 64) and at the fp32 ones (128 x 128 / 64 x 64), the LDS-DMA loader (K a multiple
    of the K step) and the register-staged one."""
    ops = _ops()
    a = _rand((M, K), dtype, 1)
    w = _rand((N, K), dtype, 2, scale=K ** -0.5)
    b = _rand((N,), torch.float32, 3, scale=0.1)
    print(f"linear dtype={dtype} out={out_dtype} M={M} N={N} K={K}", flush=True)
    out = ops.linear(a.to(gpu), w.to(gpu), b.to(gpu), out_dtype=out_dtype)
    assert out.dtype == out_dtype
    out = out.cpu().double()
    a64, w64, b64 = a.double(), w.double(), b.double()
    ref = a64 @ w64.T + b64
    bound = UNIT[out_dtype] * ref.abs() + 4 * K * 2.0 ** -24 * (a64.abs() @ w64.abs().T) + 1e-7
    err = (out - ref).abs()
    assert _report("linear", err, bound) <= 1.0


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("inplace", [False, True])
def test_linear_persistent_held_weights_and_residual(gpu, out_dtype, inplace):
    """The persistent kernel on a one-column problem whose K is one ring turn (300000 x 128 x
    128: 1172 tiles, W's stages held in the ring after the first tile) with the residual in its
    epilogue (requested two chunks at a time; in place: R is C), against fp64, and the row mask
    with zeroed rows."""
    ops = _ops()
    M, N, K = 300000, 128, 128
    a = _rand((M, K), torch.float16, 11)
    w = _rand((N, K), torch.float16, 12, scale=K ** -0.5)
    b = _rand((N,), torch.float32, 13, scale=0.1)
    r = _rand((M, N), out_dtype, 14)
    rows = torch.rand(M, generator=torch.Generator().manual_seed(15)) > 0.2
    print(f"persistent held-W linear out={out_dtype} inplace={inplace}", flush=True)
    gr = r.to(gpu)
    out = ops.linear(a.to(gpu), w.to(gpu), b.to(gpu), out_dtype=out_dtype, residual=gr,
                     out=gr if inplace else None, row_valid=rows.to(gpu), zero_masked_rows=True)
    out = out.cpu().double()
    a64, w64 = a.double(), w.double()
    proj = a64 @ w64.T + b.double()
    # the projection rounded to the output type, then the residual added and rounded again
    ref = proj + r.double()
    bound = (UNIT[out_dtype] * (proj.abs() + ref.abs()) + 4 * K * 2.0 ** -24 * (a64.abs() @ w64.abs().T)
             + 1e-7)
    err = (out - ref).abs()
    assert torch.all(out[~rows] == 0)
    assert _report("linear+residual", err[rows], bound[rows]) <= 1.0


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_linear_strided_input_and_row_mask(gpu, dtype):
    ops = _ops()
    M, N, K = 200, 96, 64
    big = _rand((M, 3 * K), dtype, 4)
    x = big[:, K:2 * K]                        # row stride 3K, unit column stride
    w = _rand((N, K), dtype, 5, scale=0.125)
    b = _rand((N,), torch.float32, 6)
    rows = torch.rand(M, generator=torch.Generator().manual_seed(7)) > 0.3
    out = ops.linear(big.to(gpu)[:, K:2 * K], w.to(gpu), b.to(gpu), row_valid=rows.to(gpu)).cpu()
    ref = x.double() @ w.double().T + b.double()
    assert torch.all(out[~rows] == 0)
    bound = UNIT[dtype] * ref.abs() + 4 * K * 2.0 ** -24 * (x.double().abs() @ w.double().abs().T) + 1e-7
    assert ((out.double() - ref).abs()[rows] <= bound[rows]).all()


def test_linear_rejects_bad_arguments(gpu):
    ops = _ops()
    from tiktok_techjam_2026_track3_amd._lib import KernelError
    a = torch.zeros(4, 12, device=gpu, dtype=torch.float16)   # K=12 is not a multiple of 8
    w = torch.zeros(8, 12, device=gpu, dtype=torch.float16)
    with pytest.raises(KernelError):
        ops.linear(a, w)
    with pytest.raises(ValueError):
        ops.linear(a, torch.zeros(8, 16, device=gpu, dtype=torch.float16))


# ---------------------------------------------------------------------------- attention
def _attn_check(gpu, dtype, B, H, Sq, Sk, hd, causal, key_valid=None, packed=False, seed=0, qscale=1.0,
                key_bound=None, kscale=1.0):
    ops = _ops()
    print(f"attention dtype={dtype} B={B} H={H} Sq={Sq} Sk={Sk} hd={hd} causal={causal} "
          f"mask={key_valid is not None} packed={packed} key_bound={key_bound}", flush=True)
    if packed:
        assert Sq == Sk
        qkv = _rand((B, Sq, 3, H, hd), dtype, seed)
        qkv[:, :, 0] = (qkv[:, :, 0].float() * qscale).to(dtype)
        g_qkv = qkv.to(gpu)
        q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
        gq, gk, gv = g_qkv[:, :, 0], g_qkv[:, :, 1], g_qkv[:, :, 2]
    else:
        q = _rand((B, Sq, H, hd), dtype, seed, scale=qscale)
        k = _rand((B, Sk, H, hd), dtype, seed + 1, scale=kscale)
        v = _rand((B, Sk, H, hd), dtype, seed + 2)
        gq, gk, gv = q.to(gpu), k.to(gpu), v.to(gpu)
    kv = None if key_valid is None else key_valid.to(gpu)
    out = ops.attention(gq, gk, gv, scale=hd ** -0.5, causal=causal, key_valid=kv,
                        key_bound=key_bound).cpu().double()
    tq, tk, tv = (t.double().transpose(1, 2) for t in (q, k, v))
    ref = OA.attention_core(tq, tk, tv, hd ** -0.5, causal, key_valid).transpose(1, 2)
    pav = OA.attention_core(tq, tk, tv.abs(), hd ** -0.5, causal, key_valid).transpose(1, 2)
    up = UNIT[dtype] if dtype != torch.float32 else 2.0 ** -22
    c = hd ** -0.5 * 1.4426950408889634
    # the exp2 argument s*c - m carries an fp32 rounding error relative to its largest
    # magnitude: allow 2^-22 * max|logit2| relative error on every probability
    logit2 = (tq @ tk.transpose(-2, -1)).abs().max().item() * c
    # the kernel rounds c*q back to the input dtype: |d s*c| <= u_in * c * (|q|.|k|) per score
    qk_abs = (tq.abs() @ tk.abs().transpose(-2, -1)).amax(dim=-1, keepdim=True).transpose(1, 2)
    uq = UNIT[dtype] if dtype != torch.float32 else 0.0
    rel = 2 * up + 2.0 ** -18 + 2.0 ** -22 * logit2 + 2 * math.log(2) * uq * c * qk_abs
    if dtype == torch.float16 and hd in (32, 64):
        # the MFMA kernel sums a sub-tile's 32 rounded fp16 probabilities per lane in a 4-level
        # tree of packed fp16 adds: the row sum, and so the whole output row, carries up to 4
        # more fp16 roundings of relative error
        rel = rel + 4 * UNIT[dtype]
    bound = rel * pav + UNIT[dtype] * ref.abs() + 1e-7
    finite = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(out), finite)
    err = (out - ref).abs()[finite]
    assert _report("attention", err, bound[finite]) <= 1.0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("S", [1, 63, 128, 200, 1000])
def test_attention_16bit(gpu, dtype, hd, causal, S):
    _attn_check(gpu, dtype, 2, 3, S, S, hd, causal)


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("S", [1, 50, 128, 300])
def test_attention_fp32(gpu, hd, causal, S):
    _attn_check(gpu, torch.float32, 2, 2, S, S, hd, causal)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_packed_qkv_views(gpu, dtype, causal):
    _attn_check(gpu, dtype, 2, 4, 333, 333, 64, causal, packed=True, seed=11)


@pytest.mark.parametrize("hd", [32, 64, 128])
def test_attention_output_rows_8_byte_aligned(gpu, hd):
    """Output rows that are only 8-byte aligned (a view 4 fp16 elements into its buffer) take
    the direct 8-byte stores instead of the LDS-staged 16-byte row chunks; both give the same
    bits."""
    ops = _ops()
    B, S, H = 2, 300, 2
    q, k, v = (_rand((B, S, H, hd), torch.float16, 70 + i).to(gpu) for i in range(3))
    aligned = ops.attention(q, k, v, scale=hd ** -0.5)
    buf = torch.full((B * S * H * hd + 4,), float("nan"), dtype=torch.float16, device=gpu)
    shifted = buf[4:].view(B, S, H, hd)
    assert shifted.data_ptr() % 16 == 8
    ops.attention(q, k, v, out=shifted, scale=hd ** -0.5)
    assert torch.equal(shifted, aligned)
    assert torch.isnan(buf[:4]).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_attention_rectangular_and_large_scores(gpu, dtype):
    _attn_check(gpu, dtype, 1, 2, 100, 700, 64, False, seed=21)
    # large logits exercise the lazy max update (tile maxima grow by more than the threshold)
    _attn_check(gpu, dtype, 1, 2, 256, 640, 64, False, seed=22, qscale=6.0)
    _attn_check(gpu, dtype, 1, 2, 256, 256, 64, True, seed=23, qscale=6.0)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_key_mask(gpu, dtype, causal):
    B, S = 3, 150
    g = torch.Generator().manual_seed(5)
    mask = torch.rand(B, S, generator=g) > 0.25
    mask[:, 0] = True                         # every causal row keeps at least key 0
    mask[2] = torch.arange(S) < 77            # a prefix mask (the benchmark's padding form)
    _attn_check(gpu, dtype, B, 2, S, S, 64, causal, key_valid=mask, seed=31)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hd", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_short_queries_key_mask(gpu, dtype, hd, causal):
    """S_q <= 128 with at least 256 (batch, head) pairs runs 128-query work-groups (half the
    waves of the regular instance): key mask with a prefix row, and (non-causal) a key range
    longer than the query range."""
    B, H, S = 8, 32, 128
    g = torch.Generator().manual_seed(hd + causal)
    mask = torch.rand(B, S, generator=g) > 0.3
    mask[:, 0] = True
    mask[2] = torch.arange(S) < 41
    _attn_check(gpu, dtype, B, H, S, S, hd, causal, key_valid=mask, seed=61)
    _attn_check(gpu, dtype, B, H, 77, 77, hd, causal, seed=63)
    if not causal:
        _attn_check(gpu, dtype, 4, 64, 96, 300, hd, False, seed=62)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_attention_fully_masked_batch_gives_nan(gpu, dtype):
    ops = _ops()
    q = torch.randn(2, 70, 1, 64, dtype=dtype, device=gpu)
    mask = torch.ones(2, 70, dtype=torch.bool, device=gpu)
    mask[1] = False
    out = ops.attention(q, q, q, key_valid=mask).cpu()
    assert torch.isfinite(out[0]).all() and torch.isnan(out[1]).all()


def test_attention_rejects_unsupported_head_dim(gpu):
    ops = _ops()
    from tiktok_techjam_2026_track3_amd._lib import KernelError
    q = torch.zeros(1, 8, 1, 40, dtype=torch.float16, device=gpu)
    with pytest.raises(KernelError, match="head_dim"):
        ops.attention(q, q, q)


# head dims of the vector-ALU kernel: 8 (2 lanes per query), 16-96 (4 lanes), 192 and 256
# (8 lanes); the benchmark's official shapes use 8, 32 and 256 (Project/shapes.json)
VALU_HDS = [8, 16, 32, 48, 80, 96, 192, 256]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hd", VALU_HDS)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("S", [1, 37, 300])
def test_attention_other_head_dims(gpu, dtype, hd, causal, S):
    _attn_check(gpu, dtype, 2, 2, S, S, hd, causal, seed=hd + S)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hd", [8, 32, 64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_short_keys_many_tiles(gpu, dtype, hd, causal):
    """Up to 256 keys and at least 1024 query tiles: the vector-ALU kernel splits each tile's
    keys over 2 waves instead of 8 (B 48, H 8, S 100: 1536 to 4992 tiles), with and without a
    key mask, and on packed q/k/v views (the strides the model passes). fp32 head dims 64 and
    128 take this path in production (official shapes 9 and 10); 16-bit 64 / 128 run the MFMA
    kernel at the same shapes."""
    B, S = 48, 100
    g = torch.Generator().manual_seed(hd + 7)
    mask = torch.rand(B, S, generator=g) > 0.2
    mask[:, 0] = True
    _attn_check(gpu, dtype, B, 8, S, S, hd, causal, seed=51)
    _attn_check(gpu, dtype, B, 8, S, S, hd, causal, key_valid=mask, seed=52)
    _attn_check(gpu, dtype, B, 8, S, S, hd, causal, packed=True, seed=53)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("hd", [32, 64])
@pytest.mark.parametrize("S", [256, 257])
def test_attention_key_split_switch_point(gpu, dtype, hd, S):
    """Both sides of the vector-ALU kernel's 2-wave / 8-wave key split (at most 256 keys and at
    least 1024 query tiles take 2 waves): S = 256 and S = 257 with enough tiles."""
    B = 64 if hd == 32 else 128
    _attn_check(gpu, dtype, B, 4, S, S, hd, False, seed=S + hd)
    _attn_check(gpu, dtype, B, 4, S, S, hd, True, seed=S + hd + 1)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("hd", [8, 32, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_other_head_dims_masked_packed(gpu, dtype, hd, causal):
    B, S = 3, 130
    g = torch.Generator().manual_seed(hd)
    mask = torch.rand(B, S, generator=g) > 0.3
    mask[:, 0] = True
    mask[1] = torch.arange(S) < 45
    _attn_check(gpu, dtype, B, 4, S, S, hd, causal, key_valid=mask, seed=41)
    _attn_check(gpu, dtype, 2, 4, S, S, hd, causal, packed=True, seed=42)
    _attn_check(gpu, dtype, 1, 2, 70, 400, hd, False, seed=43, qscale=6.0)


# --------------------------------------------------------------------------------- int8
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("K", [512, 4096, 4000, 8192, 16384, 32768])
def test_quant_rows_bit_exact(gpu, dtype, mode, K):
    """Row lengths that keep the row in registers (64 * 2^i 16-byte chunks up to 16 per lane:
    512 and 4096, 8192 16-bit) and that take the two-pass kernel (4000; 16384 and 32768 16-bit,
    8192 and more fp32)."""
    ops = _ops()
    x = _rand((300, K), dtype, 41, scale=0.7)
    x[3] = 0                                   # zero row exercises the clamp
    x[4, :16] = torch.tensor([2.5, -2.5, 0.5, 1.5] * 4, dtype=dtype)
    q, s = ops.quant_rows_i8(x.to(gpu), mode=mode)
    if mode == 0:
        wq, ws = OI.quant_rows(x.float().numpy())
    else:
        wq, ws = OI.quant_weight(x.float().numpy())
    np.testing.assert_array_equal(s.cpu().numpy(), ws)
    np.testing.assert_array_equal(q.cpu().numpy(), wq)


@pytest.mark.parametrize("M,N,K", [(1, 32, 16), (257, 300, 512), (1024, 1536, 4096), (4096, 4096, 4096)])
def test_gemm_i8_accumulators_bit_exact(gpu, M, N, K):
    ops = _ops()
    rng = np.random.default_rng(M + N + K)
    a = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    w = rng.integers(-128, 128, size=(N, K), dtype=np.int8)
    a[0, :] = -128
    w[0, :] = -128                             # extreme accumulator K * 128^2
    acc = torch.empty(M, N, dtype=torch.int32, device=gpu)
    ga, gw = torch.from_numpy(a).to(gpu), torch.from_numpy(w).to(gpu)
    ones_a = torch.ones(M, device=gpu)
    ones_w = torch.ones(N, device=gpu)
    ops.linear_i8(ga, gw, ones_a, ones_w, acc_out=acc, want_out=False)
    np.testing.assert_array_equal(acc.cpu().numpy(), OI.int8_gemm(a, w))


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32, torch.bfloat16])
def test_gemm_i8_dequant_bit_exact(gpu, out_dtype):
    ops = _ops()
    M, N, K = 300, 520, 1024
    h = _rand((M, K), torch.float32, 51)
    w = _rand((N, K), torch.float32, 52, scale=0.02)
    bias = _rand((N,), torch.float32, 53, scale=0.03)
    a8, sa = OI.quant_rows(h.numpy())
    w8, sw = OI.quant_weight(w.numpy())
    want32, _ = OI.int8_linear(h.numpy(), w8, sw, bias.numpy())
    out = ops.linear_i8(torch.from_numpy(a8).to(gpu), torch.from_numpy(w8).to(gpu),
                        torch.from_numpy(sa).to(gpu), torch.from_numpy(sw).to(gpu), bias.to(gpu),
                        out_dtype=out_dtype).cpu()
    want = torch.from_numpy(want32).to(out_dtype)
    assert torch.equal(out, want)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_attention_key_mask_repeatable(gpu, dtype):
    """The masked case above, repeated: every run must give bit-identical, correct output (a
    loader variant that reloaded spilled offsets returned wrong rows for one wave now and then)."""
    ops = _ops()
    B, S, H, hd = 3, 150, 2, 64
    g = torch.Generator().manual_seed(5)
    mask = torch.rand(B, S, generator=g) > 0.25
    mask[:, 0] = True
    mask[2] = torch.arange(S) < 77
    q, k, v = (_rand((B, S, H, hd), dtype, 31 + i).to(gpu) for i in range(3))
    ref = OA.attention_core(*(t.double().cpu().transpose(1, 2) for t in (q, k, v)), hd ** -0.5,
                            False, mask).transpose(1, 2)
    first = None
    for rep in range(12):
        out = torch.full((B, S, H, hd), float("nan"), dtype=dtype, device=gpu)
        ops.attention(q, k, v, out=out, scale=hd ** -0.5, key_valid=mask.to(gpu))
        o = out.cpu()
        assert (o.double() - ref).abs().max().item() <= 0.02, f"run {rep}"
        if first is None:
            first = o
        assert torch.equal(o, first), f"run {rep} differs from run 0"


# ------------------------------------------------------------- key-norm bound (workspace path)
def _bound_pair(gpu, dtype, B, H, S, hd, causal, scale_qk, seed, key_valid=None, packed=False):
    """The same problem through mi355_attn_fwd (exact row maxima on every tile) and
    mi355_attn_fwd_ws (key-norm bounds); returns both outputs and the inputs."""
    ops = _ops()
    if packed:
        qkv = _rand((B, S, 3, H, hd), dtype, seed, scale=scale_qk).to(gpu)
        q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    else:
        q = _rand((B, S, H, hd), dtype, seed, scale=scale_qk).to(gpu)
        k = _rand((B, S, H, hd), dtype, seed + 1, scale=scale_qk).to(gpu)
        v = _rand((B, S, H, hd), dtype, seed + 2).to(gpu)
    kv = None if key_valid is None else key_valid.to(gpu)
    a = ops.attention(q, k, v, causal=causal, key_valid=kv, key_bound=False)
    b = ops.attention(q, k, v, causal=causal, key_valid=kv, key_bound=True)
    return a.cpu(), b.cpu()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hd", [32, 64, 128])
@pytest.mark.parametrize("causal,S,scale_qk", [(False, 1100, 3.0), (True, 1100, 3.0)])
def test_attention_key_bound_bit_identical(gpu, dtype, hd, causal, S, scale_qk):
    """Without a key mask, scores within +-8 take the max-free sweep and larger ones the offset
    sweep; large scores (Q, K ~ N(0, 9)) are estimated from the first sub-tile to fail the
    offset sweep's check, so their waves keep the exact running max: the exact path's bits.
    (The bit-identical skipping of row maxima once mu can no longer move is checked on the
    key-masked launches, test_attention_key_bound_masked_packed.)"""
    sc = hd ** -0.5 if scale_qk is None else scale_qk
    print(f"key bound dtype={dtype} hd={hd} causal={causal} S={S} scale={sc}", flush=True)
    a, b = _bound_pair(gpu, dtype, 2, 3, S, hd, causal, sc, 41)
    assert torch.equal(torch.isnan(a), torch.isnan(b)) and not torch.isnan(a).any()
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hd", [32, 64, 128])
@pytest.mark.parametrize("S", [100, 256, 300, 2600, 4097])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_max_free_sweep_against_oracle(gpu, dtype, hd, S, causal):
    """Non-causal Q, K ~ N(0,1)/sqrt(head_dim) (the C5 core distribution): the key-norm bound
    puts every score within +-8 (log2 units), so the waves run the max-free sweep (mu = 0, no
    row maxima; its branch-free full stages -- causal: those before the work-group's first
    query -- then the generic stages for the tail). Checked against the oracle under the exact
    path's error bound, at lengths with no full stage, exact stages, and a partial last
    sub-tile."""
    sc = hd ** -0.5
    _attn_check(gpu, dtype, 2, 3, S, S, hd, causal, seed=45, qscale=sc, kscale=sc, key_bound=True)


def test_attention_max_free_sweep_packed_and_mixed_heads(gpu):
    """Packed QKV views in the max-free sweep against the oracle; and a head whose keys are
    large (bound far above 8 + 256: neither sweep, the exact path) beside heads in the max-free
    sweep: the large head is bit for bit the exact path's, the others within the oracle bound."""
    _attn_check(gpu, torch.float16, 2, 2, 1300, 1300, 64, False, packed=True, seed=48, qscale=0.125,
                key_bound=True)
    ops = _ops()
    B, S, H, hd = 1, 3000, 3, 64
    q = _rand((B, S, H, hd), torch.float16, 71, scale=0.125)
    k = _rand((B, S, H, hd), torch.float16, 72, scale=0.125)
    k[:, :, 2] = (k[:, :, 2].float() * 2000).half()
    v = _rand((B, S, H, hd), torch.float16, 73)
    gq, gk, gv = q.to(gpu), k.to(gpu), v.to(gpu)
    a = ops.attention(gq, gk, gv, key_bound=False).cpu()
    b = ops.attention(gq, gk, gv, key_bound=True).cpu()
    assert torch.equal(a[:, :, 2], b[:, :, 2])
    ref = OA.attention_core(*(t.double().transpose(1, 2) for t in (q, k, v)), hd ** -0.5, False,
                            None).transpose(1, 2)
    err = (b.double() - ref).abs()[:, :, :2]
    assert float(err.max()) < 2e-3


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_key_bound_masked_packed(gpu, dtype, causal):
    """Key-masked launches (exact running max, row maxima skipped once mu can no longer move:
    bit for bit; key 3 of every row is invalid, so every work-group takes the key-masked
    instance) and causal packed views without a mask (against the oracle)."""
    B, S = 2, 1300
    g = torch.Generator().manual_seed(9)
    mask = torch.rand(B, S, generator=g) > 0.2
    mask[:, 0] = True
    mask[1] = torch.arange(S) < 900
    mask[:, 3] = False
    a, b = _bound_pair(gpu, dtype, B, 2, S, 64, causal, 0.125, 47, key_valid=mask)
    assert torch.equal(a, b)
    if causal:
        # causal packed views without a mask: the max-free / offset sweeps, against the oracle
        _attn_check(gpu, dtype, B, 2, S, S, 64, causal, packed=True, seed=48, qscale=0.125,
                    key_bound=True)


@pytest.mark.parametrize("bad", [float("nan"), float("inf"), 3.0e4])
def test_attention_key_bound_nonfinite_and_huge_keys(gpu, bad):
    """A NaN / inf / huge key makes the bound of its head non-finite or loose: that head runs
    the exact path, bit for bit (NaN where it gives NaN); the other head (max-free sweep) stays
    within 1e-3 of the exact path and finite."""
    ops = _ops()
    dtype = torch.float16
    B, S, H, hd = 1, 2100, 2, 64
    q = _rand((B, S, H, hd), dtype, 61, scale=0.125).to(gpu)
    k = _rand((B, S, H, hd), dtype, 62, scale=0.125)
    k[0, 1234, 1, 5] = bad
    k = k.to(gpu)
    v = _rand((B, S, H, hd), dtype, 63).to(gpu)
    a = ops.attention(q, k, v, key_bound=False).cpu()
    b = ops.attention(q, k, v, key_bound=True).cpu()
    assert torch.equal(torch.isnan(a), torch.isnan(b))
    h1a, h1b = a[:, :, 1], b[:, :, 1]
    fin = ~torch.isnan(h1a)
    assert torch.equal(h1a[fin], h1b[fin])
    assert torch.isfinite(b[:, :, 0]).all()
    assert float((a[:, :, 0].float() - b[:, :, 0].float()).abs().max()) < 1e-3


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hd", [32, 64, 128])
@pytest.mark.parametrize("S", [100, 1500, 4097])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_offset_sweep_against_oracle(gpu, dtype, hd, S, causal):
    """Q, K ~ N(0,1) (the block's projections), non-causal and causal: the bound exceeds 8, so the waves
    run the offset sweep (mu fixed at bound - 8, no row maxima); work-groups whose row sums
    pass the check keep it, the others are redone on the exact path. Checked against the oracle
    under the exact path's error bound."""
    _attn_check(gpu, dtype, 2, 3, S, S, hd, causal, seed=49, key_bound=True)


def _redo_flags_call(gpu, q, k, v, causal=False, mask=None):
    """mi355_attn_fwd_ws with a workspace of the caller's (filled with 0x7f bytes); returns the
    output and the workspace's ints after the 256-byte aligned bounds (one per 256-key chunk of
    every head: the redo flags, one per work-group of 256 queries, then the untouched fill)."""
    from tiktok_techjam_2026_track3_amd import _lib as L
    B, S, H, hd = q.shape
    kb = B * H * ((S + 255) // 256) * 4
    off = (kb + 255) // 256 * 256
    n_wg = B * H * ((S + 255) // 256)
    ws = torch.full((off + 4 * n_wg + 256,), 0x7F, device=gpu, dtype=torch.uint8)
    out = torch.empty_like(q)
    st = [L.i64_array((t.stride(0), t.stride(1), t.stride(2))) for t in (q, k, v, out)]
    rc = L.lib().mi355_attn_fwd_ws(L.dtype_code(q.dtype), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                   out.data_ptr(), B, H, S, S, hd, *st, hd ** -0.5, int(causal),
                                   None if mask is None else mask.data_ptr(),
                                   0 if mask is None else mask.stride(0),
                                   ws.data_ptr(), ws.numel(), None)
    L.check("mi355_attn_fwd_ws", rc)
    torch.cuda.synchronize()
    return out.cpu(), ws[off:].cpu().view(torch.int32), n_wg


@pytest.mark.parametrize("hd", [32, 64, 128])
def test_attention_offset_sweep_redo_flags(gpu, hd):
    """The redo flags in the workspace. Large scores (Q, K ~ N(0, 9)): the first sub-tile's
    maxima predict that the check would fail, so no wave takes the offset sweep: no flag, the
    exact path's bits. Q, K ~ N(0,1) at head_dim 64 and S = 8192: work-groups keep the offset
    sweep's results, so the output differs from the exact path's bits (their accuracy:
    test_attention_offset_sweep_against_oracle). The flags after the work-groups' are
    untouched."""
    ops = _ops()
    for scale, B, S, H in ((3.0, 2, 1500, 3), (1.0, 1, 8192, 2)):
        q = _rand((B, S, H, hd), torch.float16, 301, scale=scale).to(gpu)
        k = _rand((B, S, H, hd), torch.float16, 302, scale=scale).to(gpu)
        v = _rand((B, S, H, hd), torch.float16, 303).to(gpu)
        exact = ops.attention(q, k, v, key_bound=False).cpu()
        out, flags, n_wg = _redo_flags_call(gpu, q, k, v)
        print(f"hd={hd} scale={scale}: {int(flags[:n_wg].sum())} of {n_wg} work-groups redone",
              flush=True)
        assert torch.all(flags[n_wg:] == 0x7F7F7F7F)
        assert torch.all((flags[:n_wg] == 0) | (flags[:n_wg] == 1))
        if scale == 3.0:
            assert torch.all(flags[:n_wg] == 0)
            assert torch.equal(out, exact)
        elif hd == 64:
            assert torch.any(flags[:n_wg] == 0)
            assert not torch.equal(out, exact)


@pytest.mark.parametrize("hd", [32, 64, 128])
def test_attention_offset_sweep_failed_check_is_redone(gpu, hd):
    """A problem built so that the prediction passes and the check fails: every query points
    along one unit vector u (|q| = sqrt(head_dim)); key 0 has norm L at cosine `cos` to u, so
    the first sub-tile's maximum a0 = cos * |cq| * L lies 2 (log2 units) below mu0 =
    1.0078 |cq| L + 1/128 - T (T = 11, the non-causal sweeps' largest exponent), within
    log2(S / 64) - 2 of it, and every other key is tiny (N(0, 0.01^2)), so the row sums come to
    about 2^(a0 - mu0) = 1/4 < 1. Every work-group is flagged, and the redo launch gives the
    exact path's bits."""
    ops = _ops()
    B, S, H, T = 1, 4096, 2, 11.0
    c = hd ** -0.5 * 1.4426950408889634
    g = torch.Generator().manual_seed(307)
    u = torch.randn(hd, generator=g)
    u = u / u.norm()
    w = torch.randn(hd, generator=g)
    w = w - (w @ u) * u
    w = w / w.norm()
    qn = hd ** 0.5
    L = 60.0 / (c * qn)                                    # |cq| L = 60: bound ~ 60.5
    cos = (60.0 * (1 + 1 / 128) + 1 / 128 - T - 2.0) / 60.0   # a0 = mu0 - 2 ~ 47.5
    q = (u * qn).expand(B, S, H, hd).clone().half()
    k = (torch.randn(B, S, H, hd, generator=g) * 0.01)
    k[:, 0] = L * (cos * u + (1 - cos ** 2) ** 0.5 * w)
    k = k.half()
    v = torch.randn(B, S, H, hd, generator=g).half()
    q, k, v = q.to(gpu), k.to(gpu), v.to(gpu)
    exact = ops.attention(q, k, v, key_bound=False).cpu()
    out, flags, n_wg = _redo_flags_call(gpu, q, k, v)
    print(f"hd={hd}: {int(flags[:n_wg].sum())} of {n_wg} work-groups redone", flush=True)
    assert torch.all(flags[:n_wg] == 1)
    assert torch.equal(out, exact)


# ------------------------------------------------------------ all-true key mask (device check)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hd", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("S", [1, 17, 130, 1000, 2053])
def test_attention_all_true_mask_same_bits(gpu, dtype, hd, causal, S):
    """A key mask that is all true over a work-group's keys is recognised on the device (one
    scan of the row's bytes), after which the sweep runs as without a mask: the same bits as
    the call without a mask, for row lengths that leave misaligned heads and byte tails."""
    ops = _ops()
    print(f"all-true mask dtype={dtype} hd={hd} causal={causal} S={S}", flush=True)
    B, H = 2, 2
    q = _rand((B, S, H, hd), dtype, 81).to(gpu)
    k = _rand((B, S, H, hd), dtype, 82).to(gpu)
    v = _rand((B, S, H, hd), dtype, 83).to(gpu)
    mask = torch.ones(B, S, dtype=torch.bool, device=gpu)
    a = ops.attention(q, k, v, causal=causal, key_valid=mask)
    b = ops.attention(q, k, v, causal=causal)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("pos", [0, 5, 16, 1024, 2040, 2052])
def test_attention_single_invalid_key_is_seen(gpu, dtype, causal, pos):
    """One invalid key anywhere in a row (the misaligned head, the 16-byte body, the byte tail;
    row stride 2053 bytes, so the second row starts misaligned) must switch that work-group back
    to the masked sweep: checked against the oracle; the other row is all true."""
    B, S = 2, 2053
    mask = torch.ones(B, S, dtype=torch.bool)
    mask[1, pos] = False   # (causal, pos 0: query 0 of row 1 has no valid key, NaN as in the oracle)
    _attn_check(gpu, dtype, B, 2, S, S, 64, causal, key_valid=mask, seed=91)


# ---------------------------------------- key mask with the bound workspace (resolved on the device)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("scale", [0.125, 1.0])
def test_attention_mask_resolved_on_device(gpu, dtype, causal, scale):
    """A key mask with the bound workspace: row 0 all true, row 1 with one invalid key at 1700
    (S = 3000). Work-groups whose keys are all valid run the unmasked instance (max-free sweep
    at scale 0.125, offset sweep at 1.0): row 0, and in causal launches row 1's query tiles
    that end before the invalid key (rows [0, 1536)), have the bits of the call without a mask.
    The others are run by the key-masked redo launch: the bits of the key-masked call without
    the workspace (exact running max). The whole output is checked against the oracle too."""
    ops = _ops()
    B, S, H, hd = 2, 3000, 2, 64
    print(f"mask on device dtype={dtype} causal={causal} scale={scale}", flush=True)
    q = _rand((B, S, H, hd), dtype, 501, scale=scale).to(gpu)
    k = _rand((B, S, H, hd), dtype, 502, scale=scale).to(gpu)
    v = _rand((B, S, H, hd), dtype, 503).to(gpu)
    mask = torch.ones(B, S, dtype=torch.bool)
    mask[1, 1700] = False
    m = mask.to(gpu)
    out = ops.attention(q, k, v, causal=causal, key_valid=m, key_bound=True).cpu()
    unmasked = ops.attention(q, k, v, causal=causal, key_bound=True).cpu()
    masked_exact = ops.attention(q, k, v, causal=causal, key_valid=m, key_bound=False).cpu()
    assert torch.equal(out[0], unmasked[0])
    split = 1536 if causal else 0
    assert torch.equal(out[1, :split], unmasked[1, :split])
    assert torch.equal(out[1, split:], masked_exact[1, split:])
    _attn_check(gpu, dtype, B, H, S, S, hd, causal, key_valid=mask, seed=501, qscale=scale,
                kscale=scale, key_bound=True)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_mask_check_redo_flags(gpu, causal):
    """The redo flags of a masked call with the workspace (Q, K ~ N(0,1)/8: the max-free sweep,
    whose results are never redone): exactly the work-groups that visit an invalid key are
    flagged. Row 0 has its only invalid key at 600 (causal: query tiles 2.. visit it), row 1 is
    all true; B = 2, H = 2, S = 2000 (8 query tiles per head)."""
    B, S, H, hd = 2, 2000, 2, 64
    q = _rand((B, S, H, hd), torch.float16, 511, scale=0.125).to(gpu)
    k = _rand((B, S, H, hd), torch.float16, 512, scale=0.125).to(gpu)
    v = _rand((B, S, H, hd), torch.float16, 513).to(gpu)
    mask = torch.ones(B, S, dtype=torch.bool)
    mask[0, 600] = False
    out, flags, n_wg = _redo_flags_call(gpu, q, k, v, causal=causal, mask=mask.to(gpu))
    nt = (S + 255) // 256
    # the work-group of (b, h, query tile qt): causal grids run the last query tiles first
    # (linear index ((nt - 1 - qt) * B + b) * H + h); non-causal grids deal (b, h, qt) to the
    # 8 XCDs (flag order does not matter here: count per batch row)
    flags = flags[:n_wg]
    if causal:
        want = torch.zeros(n_wg, dtype=torch.int32)
        for qt in range(nt):
            for b in range(B):
                for h in range(H):
                    lin = ((nt - 1 - qt) * B + b) * H + h
                    want[lin] = int(b == 0 and (qt + 1) * 256 > 600)
        assert torch.equal(flags, want)
    else:
        assert int(flags.sum()) == H * nt              # every work-group of batch row 0
    ref = OA.attention_core(*(t.cpu().double().transpose(1, 2) for t in (q, k, v)), hd ** -0.5,
                            causal, mask).transpose(1, 2)
    assert float((out.double() - ref).abs().max()) < 2e-3


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hd", [32, 64, 128])
@pytest.mark.parametrize("scale", [0.125, 1.0])
def test_attention_causal_rows_ignore_later_tokens(gpu, dtype, hd, scale):
    """Causal calls with the bound workspace at a length where work-groups take the sweeps
    (S = 34816: query tiles whose key range reaches 32768 keys run the max-free sweep at scale
    0.125 and the offset sweep at 1.0): the output of a 256-row query tile depends on no token
    after the tile. Replacing every query, key and value from token 34000 on leaves rows
    [0, 33792) (the tiles that end at or before token 34000) bit for bit unchanged; a call on
    the first 33792 tokens alone gives those rows bit for bit; and with the library's default
    workspace choice a 2048-token prefix (no workspace: the exact running max) gives the first
    2048 rows of the full-length call (workspace) bit for bit, since tiles shorter than 32768
    keys never take the sweeps."""
    ops = _ops()
    B, S, H, P, R = 1, 34816, 2, 34000, 33792
    print(f"causal tiles dtype={dtype} hd={hd} scale={scale}", flush=True)
    q, k, v = (_rand((B, S, H, hd), dtype, 521 + i, scale=scale if i < 2 else 1.0).to(gpu)
               for i in range(3))
    full = ops.attention(q, k, v, causal=True, key_bound=True)
    q2, k2, v2 = (t.clone() for t in (q, k, v))
    for i, t in enumerate((q2, k2, v2)):
        t[:, P:] = _rand((B, S - P, H, hd), dtype, 531 + i, scale=4.0).to(gpu)
    changed = ops.attention(q2, k2, v2, causal=True, key_bound=True)
    assert torch.equal(full[:, :R], changed[:, :R])
    head = ops.attention(*(t[:, :R].contiguous() for t in (q, k, v)), causal=True, key_bound=True)
    assert torch.equal(head, full[:, :R])
    default_full = ops.attention(q, k, v, causal=True)
    default_head = ops.attention(*(t[:, :2048].contiguous() for t in (q, k, v)), causal=True)
    assert torch.equal(default_head, default_full[:, :2048])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hd", [32, 64, 128])
@pytest.mark.parametrize("scale", [0.125, 1.0])
def test_attention_causal_sweeps_long_against_reference(gpu, dtype, hd, scale):
    """Causal attention at S = 33280 with the library's default workspace (the last two query
    tiles' key ranges reach 32768 keys: max-free sweep at scale 0.125, offset sweep at 1.0, the
    redo launch), sampled rows against an fp64 evaluation of the same rounded inputs, under the
    error bound of the exact path (module docstring; the fp16 row-sum tree adds its 4
    roundings)."""
    ops = _ops()
    B, S, H = 1, 33280, 2
    print(f"causal long dtype={dtype} hd={hd} scale={scale}", flush=True)
    q = _rand((B, S, H, hd), dtype, 541, scale=scale)
    k = _rand((B, S, H, hd), dtype, 542, scale=scale)
    v = _rand((B, S, H, hd), dtype, 543)
    out = ops.attention(q.to(gpu), k.to(gpu), v.to(gpu), causal=True).cpu().double()
    g = torch.Generator().manual_seed(544)
    idx = torch.tensor(sorted(set([0, 255, 32511, 32512, 32767, 32768, 33023, 33024, 33279]
                                  + torch.randint(32512, S, (24,), generator=g).tolist())))
    tq = q[0, idx].double().transpose(0, 1)                  # [H, n, hd]
    tk, tv = (t[0].double().transpose(0, 1) for t in (k, v))  # [H, S, hd]
    c = hd ** -0.5 * 1.4426950408889634
    s = (tq @ tk.transpose(-2, -1)) * hd ** -0.5              # [H, n, S]
    s = s.masked_fill(torch.arange(S)[None, None, :] > idx[None, :, None], float("-inf"))
    p = torch.softmax(s, dim=-1)
    ref = (p @ tv).transpose(0, 1)                            # [n, H, hd]
    pav = (p @ tv.abs()).transpose(0, 1)
    logit2 = float((tq @ tk.transpose(-2, -1)).abs().max()) * c
    qk_abs = (tq.abs() @ tk.abs().transpose(-2, -1)).amax(dim=-1, keepdim=True).transpose(0, 1)
    up = UNIT[dtype]
    rel = 2 * up + 2.0 ** -18 + 2.0 ** -22 * logit2 + 2 * math.log(2) * up * c * qk_abs
    if dtype == torch.float16 and hd in (32, 64):
        rel = rel + 4 * UNIT[dtype]
    bound = rel * pav + UNIT[dtype] * ref.abs() + 1e-7
    err = (out[0, idx] - ref).abs()
    assert _report("causal long sampled rows", err, bound) <= 1.0


@pytest.mark.parametrize("masked", [False, True])
def test_attention_long_graph_capture_equals_eager(gpu, masked):
    """A SelfAttention forward at a key length with the bound workspace (S = 40000, the C5
    block's d_model 512 and 8 heads) captured in a HIP graph: replays equal the eager forward
    bit for bit, with the all-true mask and with one whose row 1 has an invalid key (eager and
    captured calls take the same kernels; nothing in the forward reads the mask on the host)."""
    from tiktok_techjam_2026_track3_amd import SelfAttention
    torch.manual_seed(77)
    mod = SelfAttention(512, 8).to(device=gpu, dtype=torch.float16)
    B, S = 2, 40000
    x = torch.randn(B, S, 512, device=gpu).half()
    mask = torch.ones(B, S, dtype=torch.bool, device=gpu)
    if masked:
        mask[1, 31000] = False
    with torch.inference_mode():
        eager = mod(x, mask)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            mod(x, mask)
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = mod(x, mask)
        for rep in range(3):
            out.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {rep}"
            mod(x[:1], mask[:1])        # eager work between the replays


@pytest.mark.parametrize("K", [64, 1024, 4096])
def test_layer_norm_fp32_to_fp16_is_the_rounded_fp32_result(gpu, K):
    """mi355_layernorm_cvt fp32 -> fp16: the same fp32 computation as the fp32 LayerNorm kernel,
    rounded once to fp16 (round to nearest even, as torch's .half())."""
    ops = _ops()
    M = 300
    x = _rand((M, K), torch.float32, 101, scale=3.0)
    x[5] += 100.0                                  # a row with a large mean
    w = _rand((K,), torch.float32, 102)
    b = _rand((K,), torch.float32, 103)
    xg, wg, bg = x.to(gpu), w.to(gpu), b.to(gpu)
    y32 = ops.layer_norm(xg, wg, bg, 1e-5)
    y16 = ops.layer_norm(xg, wg, bg, 1e-5, out_dtype=torch.float16)
    assert y16.dtype == torch.float16
    assert torch.equal(y16, y32.half())
