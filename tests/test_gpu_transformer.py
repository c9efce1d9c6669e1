"""GPU parity of the rest of the transformer block and model (torch_transformer_benchmark.py:
125-172) on the gfx950 kernels: the GELU and zero-masked residual epilogues, the masked
LayerNorm, TransformerBlock / Transformer and the plugin's full-model path.

Bars:
* GELU epilogue: against ``gelu(plain)`` where ``plain`` is the same kernel's output without the
  GELU (so the GEMM is not re-judged here) -- within one unit in the last place of the output
  dtype of torch's fp32 formula x * 0.5 * (1 + erf(x / sqrt 2)) (the reference's arithmetic,
  which cancels for negative x: ~2e-5 relative at x = -3), and at least 99% of 16-bit elements
  bit-identical to the GELU computed in fp64 and rounded; fp32 outputs within 4 fp32 ulps plus
  3e-7 absolute of torch's formula and 4e-7 absolute of fp64.
* zero-masked residual epilogue and masked LayerNorm: bit-exact against the unmasked kernels'
  output on valid rows, exact zeros on masked rows.
* block / model: the benchmark's elementwise predicate (oracle.predicate) against the oracle in
  fp32 (fp32, fp16); bf16 against the oracle with the bf16 model's rounding points, each stage
  judged on the kernel's own input, widened by one bf16 unit in the last place of the rounded
  intermediates that enter the output additively.
"""
import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import block as OB
from oracle import int8 as OI
from oracle import model as OM
from oracle.predicate import compare_outputs
from tiktok_techjam_2026_track3_amd import workloads as W

pytestmark = pytest.mark.gpu

MANT = {torch.float16: 10, torch.bfloat16: 7, torch.float32: 23}


def _ulp(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    e = torch.floor(torch.log2(t.abs().double().clamp_min(torch.finfo(dtype).tiny)))
    return torch.exp2(e - MANT[dtype])


# ------------------------------------------------------------------------- GELU epilogue
GELU_CASES = [
    (torch.float16, torch.float16, 300, 520, 256), (torch.float16, torch.float16, 1024, 2048, 512),
    (torch.bfloat16, torch.bfloat16, 300, 520, 256), (torch.bfloat16, torch.bfloat16, 64, 100, 128),
    (torch.float16, torch.bfloat16, 512, 1024, 256),
    (torch.float32, torch.float32, 128, 768, 256),    # split-K small-problem kernel
    (torch.float32, torch.float32, 1200, 768, 256),   # 64 x 64 tiles
    (torch.float32, torch.float32, 4096, 1024, 256),  # 128 x 128 tiles
]


@pytest.mark.parametrize("dtype,odt,M,N,K", GELU_CASES)
def test_gelu_epilogue(gpu, dtype, odt, M, N, K):
    from tiktok_techjam_2026_track3_amd import ops
    g = torch.Generator().manual_seed(M * 7 + N + K)
    x = torch.randn(M, K, generator=g).to(dtype).to(gpu)
    w = (torch.randn(N, K, generator=g) * 2 * K ** -0.5).to(dtype).to(gpu)
    b = torch.randn(N, generator=g).to(gpu)
    print(f"gelu epilogue {dtype}->{odt} M={M} N={N} K={K}", flush=True)
    plain = ops.linear(x, w, b, out_dtype=odt)
    fused = ops.linear(x, w, b, out_dtype=odt, gelu=True)
    torch.cuda.synchronize()
    ref = OB.gelu(plain.float().cpu())          # torch's fp32 arithmetic (the reference's)
    exact = OB.gelu(plain.double().cpu())       # fp64: the correctly rounded target
    got = fused.float().cpu()
    d = (got - ref.to(odt).float()).abs()
    if odt == torch.float32:
        tol = 4 * _ulp(ref, torch.float32).float() + 3e-7
    else:
        # plus the absolute error of torch's own fp32 formula where 1 + erf cancels (it returns
        # exactly 0 below x ~ -5.5, where bf16 still holds the true, tiny value)
        tol = _ulp(ref, odt).float() + 4e-7
    bad = d > tol
    same = float((got == exact.to(odt).float()).float().mean())
    print(f"  max |d| vs torch fp32 {float(d.max()):.3g}, beyond tolerance {int(bad.sum())}; "
          f"bit-identical to the rounded fp64 GELU {same:.4f}", flush=True)
    assert not bad.any()
    if odt != torch.float32:
        assert same >= 0.99
    else:
        assert float((got.double() - exact).abs().max()) <= 4e-7
    with pytest.raises(ValueError):
        ops.linear(x, w, b, out_dtype=odt, gelu=True, residual=plain)


# ------------------------------------------------------- zero-masked residual / masked norm
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,K", [(300, 520, 256), (1024, 1024, 2048), (64, 100, 128)])
def test_residual_zero_masked_bit_exact(gpu, dtype, M, N, K):
    from tiktok_techjam_2026_track3_amd import ops
    g = torch.Generator().manual_seed(M + 3 * N + K)
    x = torch.randn(M, K, generator=g).to(dtype).to(gpu)
    w = (torch.randn(N, K, generator=g) * K ** -0.5).to(dtype).to(gpu)
    b = torch.randn(N, generator=g).to(gpu)
    r = (torch.randn(M, N, generator=g) * 2).to(dtype).to(gpu)
    valid = (torch.rand(M, generator=g) > 0.3).to(gpu)
    print(f"zero-masked residual {dtype} M={M} N={N} K={K}", flush=True)
    fused = ops.linear(x, w, b, residual=r)
    zm = ops.linear(x, w, b, residual=r, row_valid=valid, zero_masked_rows=True)
    assert torch.equal(zm[valid], fused[valid])
    assert torch.all(zm[~valid] == 0)
    assert torch.equal(ops.linear(x, w, b, residual=r, zero_masked_rows=True), fused)
    inplace = r.clone()
    ops.linear(x, w, b, residual=inplace, out=inplace, row_valid=valid, zero_masked_rows=True)
    assert torch.equal(inplace, zm)


@pytest.mark.parametrize("dtype,K", [(torch.float16, 1024), (torch.bfloat16, 2048),
                                     (torch.float32, 256), (torch.float16, 4096),
                                     (torch.float32, 128), (torch.float16, 64), (torch.float32, 32)])
def test_layer_norm_masked_rows(gpu, dtype, K):
    from tiktok_techjam_2026_track3_amd import ops
    g = torch.Generator().manual_seed(K)
    M = 517
    x = torch.randn(M, K, generator=g).to(dtype).to(gpu)
    wt = (torch.randn(K, generator=g) * 0.3 + 1).to(dtype).to(gpu)
    bs = (torch.randn(K, generator=g) * 0.1).to(dtype).to(gpu)
    valid = (torch.rand(M, generator=g) > 0.4).to(gpu)
    plain = ops.layer_norm(x, wt, bs, 1e-5)
    masked = ops.layer_norm(x, wt, bs, 1e-5, row_valid=valid)
    assert torch.equal(masked[valid], plain[valid])
    assert torch.all(masked[~valid] == 0)
    inplace = x.clone()
    ops.layer_norm(inplace, wt, bs, 1e-5, out=inplace, row_valid=valid)
    assert torch.equal(inplace, masked)


# ---------------------------------------------------------------------- block and model
def _model(cfg, dtype, gpu, seed=1234):
    from tiktok_techjam_2026_track3_amd import Transformer
    torch.manual_seed(seed)
    baseline = OM.BaselineTransformer(cfg).eval()
    with torch.no_grad():  # non-trivial norm affines (nn.LayerNorm starts at 1 / 0)
        for name, prm in baseline.named_parameters():
            if "norm" in name:
                prm.add_(0.1 * torch.randn_like(prm))
    model = Transformer(cfg)
    model.load_state_dict(baseline.state_dict(), strict=True)
    return baseline, model.to(device=gpu, dtype=dtype).eval()


def _params(module, dtype):
    return {k: v.detach().to(dtype).float() for k, v in module.state_dict().items()}


def _assert_ffn(x1, params, mask, dtype, out):
    """The FFN half of one block on the kernel's own attention-half output ``x1``."""
    if dtype != torch.bfloat16:
        ref = OB.ffn_half(x1.float(), params, mask)
        r = compare_outputs(ref, out)
        print("  ffn half:", r.summary(), flush=True)
        assert r.passed, r.summary()
        return
    ref = OB.ffn_half(x1.float(), params, mask, round_to=torch.bfloat16)
    h = OA.layer_norm(x1.float(), params["norm2.weight"], params["norm2.bias"]).to(torch.bfloat16).float()
    f = torch.nn.functional.linear(h, params["ffn_in.weight"], params["ffn_in.bias"]).to(torch.bfloat16).float()
    o = torch.nn.functional.linear(OB.gelu(f).to(torch.bfloat16).float(), params["ffn_out.weight"],
                                   params["ffn_out.bias"])
    d = (out.float() - ref).abs()
    wide = 2e-3 + _ulp(o, torch.bfloat16).float() + _ulp(ref, torch.bfloat16).float()
    ok = torch.isfinite(out.float()) & ((d <= wide) | (d <= 2e-2 * ref.abs()))
    print(f"  bf16 ffn half: max |d| {float(d.max()):.3g}, beyond the widened predicate "
          f"{int((~ok).sum())}; plain predicate: {compare_outputs(ref, out).summary()}", flush=True)
    assert ok.all()


def _assert_attention_half(h, bl, mask, causal, dtype, out, heads):
    pf = _params(bl.attention, dtype)
    wn = bl.norm1.weight.detach().to(dtype).float()
    bn = bl.norm1.bias.detach().to(dtype).float()
    if dtype != torch.bfloat16:
        ref = OA.attention_half(h.float(), wn, bn, pf, heads, mask, causal, bl.norm1.eps)
        r = compare_outputs(ref, out)
        print("  attention half:", r.summary(), flush=True)
        assert r.passed, r.summary()
        return
    ref = OA.attention_half(h.float(), wn, bn, pf, heads, mask, causal, bl.norm1.eps,
                            round_to=torch.bfloat16)
    hh = OA.layer_norm(h.float(), wn, bn, bl.norm1.eps).to(torch.bfloat16).float()
    att = OA.self_attention(hh, pf, heads, mask, causal)
    d = (out.float() - ref).abs()
    ok = torch.isfinite(out.float()) & (
        (d <= 2e-3 + _ulp(att, torch.bfloat16).float() + _ulp(ref, torch.bfloat16).float())
        | (d <= 2e-2 * ref.abs()))
    print(f"  bf16 attention half: beyond the widened predicate {int((~ok).sum())}", flush=True)
    assert ok.all()


def _check_block_by_block(gpu, cfg, dtype, lengths=None, seed=99):
    """Transformer judged block by block: each block's attention half on its own input, then
    the FFN half on the kernel's attention-half output, then the final masked norm; the block
    output equals forward_residual followed by the FFN kernels; masked rows are exact zeros.
    ``lengths`` (per batch row) makes a prefix mask; None runs without a mask. fp32 models are
    also compared end to end with the oracle transformer."""
    from tiktok_techjam_2026_track3_amd import ops
    B, S, d, causal = cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.causal
    baseline, model = _model(cfg, dtype, gpu)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, S, d, generator=g).to(dtype)
    mask = None
    if lengths is not None:
        mask = torch.arange(S)[None, :] < torch.tensor(lengths)[:, None]
        x = x.masked_fill(~mask[..., None], 0)
    mg = None if mask is None else mask.to(gpu)
    with torch.inference_mode():
        h = x.to(gpu)
        for i, (ml, bl) in enumerate(zip(model.layers, baseline.layers)):
            print(f" layer {i}", flush=True)
            x1 = ml.attention.forward_residual(h, ml.norm1, mg, causal)
            _assert_attention_half(h.cpu(), bl, mask, causal, dtype, x1.cpu(), cfg.num_heads)
            y = ml(h, mg, causal)
            fp = _params(bl, dtype)
            _assert_ffn(x1.cpu(), fp, mask, dtype, y.cpu())
            if mask is not None:
                assert torch.all(y.cpu()[~mask] == 0)
            h = y
        out = model(x.to(gpu), mg)
        fw = model.final_norm.weight.detach()
        fb = model.final_norm.bias.detach()
        want = ops.layer_norm(h.reshape(-1, d), fw, fb, model.final_norm.eps).view_as(h)
        if mask is not None:
            want = want.masked_fill(~mg[..., None], 0)
        assert torch.equal(out, want)
    if dtype == torch.float32:
        ref = baseline(x.float(), mask)
        r = compare_outputs(ref, out)
        print("end to end vs fp32 oracle transformer:", r.summary(), flush=True)
        assert r.passed, r.summary()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("masked", [False, True])
def test_transformer_matches_oracle_block_by_block(gpu, dtype, causal, masked):
    """Transformer (2 layers, d 256, 4 heads of 64)."""
    cfg = OM.TransformerConfig(batch_size=2, seq_len=320, d_model=256, num_heads=4, ffn_dim=1024,
                               num_layers=2, causal=causal)
    print(f"transformer dtype={dtype} causal={causal} masked={masked}", flush=True)
    _check_block_by_block(gpu, cfg, dtype, [320, 201] if masked else None)


# The benchmark's 14 official shapes (Project/shapes.json; every one causal), run by
# torch_transformer_benchmark.py in float32 unless --dtype says otherwise. Head dims: 32 (d128/4
# heads), 8 (d32/4, d128/16), 256 (d1024/4), 128 (d128/1), 64 (d128/2, d1024/16).
OFFICIAL_SHAPES = [(sid, *dims) for sid, dims in sorted(W.OFFICIAL_SHAPES.items())]
# (id, batch, d_model, heads, seq_len, layers, ffn_dim)


def _official_cfg(shape, max_batch, max_seq):
    _sid, B, d, H, S, L, F = shape
    return OM.TransformerConfig(batch_size=min(B, max_batch), seq_len=min(S, max_seq), d_model=d,
                                num_heads=H, ffn_dim=F, num_layers=L, causal=True)


@pytest.mark.parametrize("shape", OFFICIAL_SHAPES, ids=[f"shape{s[0]}" for s in OFFICIAL_SHAPES])
def test_official_shapes_fp32_end_to_end(gpu, shape):
    """The whole model (every layer and the final norm on the kernels) at the official shape,
    batch capped at 3 and sequence at 2048 so the CPU oracle stays fast, with the harness's
    all-true valid_token_mask (generate_random_case, torch_transformer_benchmark.py:255-259),
    judged by the reference's predicate against the fp32 oracle model."""
    cfg = _official_cfg(shape, 3, 2048)
    print(f"official shape {shape[0]}: {cfg}", flush=True)
    baseline, model = _model(cfg, torch.float32, gpu, seed=1234 + shape[0])
    g = torch.Generator().manual_seed(shape[0])
    x = torch.randn(cfg.batch_size, cfg.seq_len, cfg.d_model, generator=g)
    mask = torch.ones(cfg.batch_size, cfg.seq_len, dtype=torch.bool)
    with torch.inference_mode():
        out = model(x.to(gpu), mask.to(gpu)).cpu()
    ref = baseline(x, mask)
    r = compare_outputs(ref, out)
    print("  vs fp32 oracle:", r.summary(), flush=True)
    assert r.passed, r.summary()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_official_shape14_full_length_causal_prefix(gpu, dtype):
    """Official shape 14 at its real size (B 32, S 100000, d 1024, 16 heads, 2 layers, the
    benchmark's float32 default and float16). Every block is causal and per token elsewhere, and
    the attention kernel's choices (key-norm bounds, the max-free and offset sweeps, redo
    flags) for a 256-row query tile depend on no token after the tile, so output rows [0, P)
    for P a multiple of 256 depend only on input rows [0, P): the first 2048 rows of the
    full-length run (the library's default path: bound pass and sweeps at this length) must
    equal the same model run on the first 2048 tokens alone, bit for bit, and those are judged
    by the reference's predicate against the fp32 oracle model (fp32; the 16-bit model is
    checked block by block at this shape below). The default run is also compared with the
    exact running max (key_bound False) by the predicate on 2 x 16384 rows. Every output is
    finite, and a batch row run alone gives the same bits as in the full batch. The fp32 model
    takes fp16 projection operands only from a size on (SelfAttention.fp16_operand_min_elems),
    which the 2048-token prefix is below: the threshold is pinned to 0 so all runs take the
    full-length run's operands."""
    shape = OFFICIAL_SHAPES[13]
    cfg = _official_cfg(shape, 32, 100000)
    B, S, d, P = cfg.batch_size, cfg.seq_len, cfg.d_model, 2048
    print(f"official shape 14 full length dtype={dtype}: {cfg}", flush=True)
    baseline, model = _model(cfg, dtype, gpu, seed=1414)
    for blk in model.layers:
        blk.attention.fp16_operand_min_elems = 0
    g = torch.Generator(device=gpu).manual_seed(1414)
    x = torch.randn(B, S, d, device=gpu, generator=g).to(dtype)
    mask = torch.ones(B, S, dtype=torch.bool, device=gpu)
    rows = [0, B - 1]
    with torch.inference_mode():
        out = model(x, mask)
        assert torch.isfinite(out).all()
        alone = model(x[B - 1:B].contiguous(), mask[B - 1:B].contiguous())
        assert torch.equal(alone[0], out[B - 1])
        del alone
        # the prefix property on the default path, bit for bit
        prefix = model(x[rows, :P].contiguous(), mask[rows, :P].contiguous())
        assert torch.equal(prefix, out[rows, :P])
        # the exact running max (no key-norm bound workspace) against the default run
        for blk in model.layers:
            blk.attention.key_bound = False
        exact = model(x[rows].contiguous(), mask[rows].contiguous())
        r = compare_outputs(exact[:, :16384].float().cpu(), out[rows, :16384].float().cpu())
        print("  default vs exact running max, 2 x 16384 rows:", r.summary(), flush=True)
        assert r.passed, r.summary()
    del out, exact
    if dtype == torch.float32:
        ref = baseline(x[rows, :P].cpu(), torch.ones(len(rows), P, dtype=torch.bool))
        r = compare_outputs(ref, prefix.cpu())
        print("  first 2048 rows vs fp32 oracle:", r.summary(), flush=True)
        assert r.passed, r.summary()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("sid", [2, 7, 8, 9, 11, 12, 14])
def test_official_shapes_16bit_block_by_block(gpu, dtype, sid):
    """16-bit models at the official shapes of every head dim (32, 8, 256, 128, 8 with 16
    heads, 64 with 16 heads (shape 14), and the 32-token sequence), batch capped at 2, sequence
    at 2048, one row padded."""
    shape = OFFICIAL_SHAPES[sid - 1]
    cfg = _official_cfg(shape, 2, 2048)
    print(f"official shape {sid} dtype={dtype}: {cfg}", flush=True)
    S = cfg.seq_len
    _check_block_by_block(gpu, cfg, dtype, [S, max(1, S // 3)][:cfg.batch_size], seed=sid)


def test_official_shape6_full_batch_sampled_rows(gpu):
    """Shape 6 at its full batch of 10000 sequences (1.28M tokens, fp32): the model runs on
    every row; rows 0, 4321 and 9999 are checked against the fp32 oracle model run on those
    rows alone (the forward is independent per batch row)."""
    cfg = _official_cfg(OFFICIAL_SHAPES[5], 10000, 128)
    baseline, model = _model(cfg, torch.float32, gpu, seed=6)
    g = torch.Generator().manual_seed(606)
    x = torch.randn(cfg.batch_size, cfg.seq_len, cfg.d_model, generator=g)
    mask = torch.ones(cfg.batch_size, cfg.seq_len, dtype=torch.bool)
    with torch.inference_mode():
        out = model(x.to(gpu), mask.to(gpu)).cpu()
    rows = torch.tensor([0, 4321, 9999])
    ref = baseline(x[rows], mask[rows])
    r = compare_outputs(ref, out[rows])
    print("shape 6 full batch, sampled rows vs fp32 oracle:", r.summary(), flush=True)
    assert r.passed, r.summary()
    assert torch.isfinite(out).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_plugin_full_model_equals_transformer(gpu, dtype):
    """build(otb, config, full_model=True) and make_user_optimized_transformer(full_model=True)
    load the baseline state dict strictly and give the Transformer module's output bit for bit."""
    from tiktok_techjam_2026_track3_amd import build, make_user_optimized_transformer
    cfg = OM.TransformerConfig(batch_size=2, seq_len=256, d_model=256, num_heads=4, ffn_dim=512,
                               num_layers=2, causal=True)
    baseline, model = _model(cfg, dtype, gpu, seed=7)
    plug = build(OM, cfg, full_model=True)
    plug.load_state_dict(baseline.state_dict(), strict=True)
    plug = plug.to(device=gpu, dtype=dtype).eval()
    U = make_user_optimized_transformer(OM, full_model=True)
    user = U(cfg)
    user.load_state_dict(baseline.state_dict(), strict=True)
    user = user.to(device=gpu, dtype=dtype).eval()
    x = torch.randn(2, 256, 256, generator=torch.Generator().manual_seed(8)).to(dtype).to(gpu)
    mask = (torch.arange(256)[None, :] < torch.tensor([256, 130])[:, None]).to(gpu)
    with torch.inference_mode():
        want = model(x, mask)
        assert torch.equal(plug(x, mask), want)
        assert torch.equal(user(x, mask), want)
        assert torch.equal(model(x), plug(x))


def test_block_weight_updates_invalidate_ffn_cache(gpu):
    from tiktok_techjam_2026_track3_amd import TransformerBlock
    blk = TransformerBlock(128, 2, 256).to(device=gpu, dtype=torch.float16).eval()
    x = torch.randn(1, 64, 128, device=gpu, dtype=torch.float16)
    with torch.inference_mode():
        a = blk(x, None, False)
    with torch.no_grad():
        blk.ffn_out.weight.mul_(2.0)
    with torch.inference_mode():
        b = blk(x, None, False)
    assert not torch.equal(a, b)
    sd = {k: v.clone() for k, v in blk.state_dict().items()}
    sd["ffn_in.bias"] += 1.0
    blk.load_state_dict(sd)
    with torch.inference_mode():
        c = blk(x, None, False)
    assert not torch.equal(b, c)


# ---------------------------------------------------------------------- int8 (W8A8) block
# fraction of the whole int8 block's output elements that must pass the predicate against the
# quantised recipe (fp32 model; measured 0.989-0.992: four requantisation points)
INT8_BLOCK_PASS_FLOOR = 0.985


def _round(a, dtype):
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(dtype).float()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("causal", [False, True])
def test_int8_block_stages(gpu, dtype, causal):
    """The W8A8 block (block_forward, k008_int8_gemm.py:189-234) on the kernels, judged stage by
    stage on the kernel's own intermediates: the quantised activations (values and scales), the
    fp16 QKV, the residual sums x1 = x + out_proj and y = x1 + ffn_out (masked rows keeping x,
    then zeroed) bit for bit against the recipe's integer arithmetic; the LayerNorms and the
    attention by the reference's predicate; the GELU epilogue within 1 ulp of the exact GELU of
    the same dequantised projection."""
    from tiktok_techjam_2026_track3_amd import Transformer
    from tiktok_techjam_2026_track3_amd.transformer import block_forward
    B, S, d, H, F = 2, 200, 256, 4, 512
    cfg = OM.TransformerConfig(batch_size=B, seq_len=S, d_model=d, num_heads=H, ffn_dim=F,
                               num_layers=1, causal=causal)
    torch.manual_seed(4321)
    baseline = OM.BaselineTransformer(cfg).eval()
    with torch.no_grad():
        for name, prm in baseline.named_parameters():
            if "norm" in name:
                prm.add_(0.1 * torch.randn_like(prm))
    model = Transformer(cfg, int8=True)
    model.load_state_dict(baseline.state_dict(), strict=True)
    model = model.to(device=gpu, dtype=dtype).eval()
    blk = model.layers[0]
    g = torch.Generator().manual_seed(17)
    x = torch.randn(B, S, d, generator=g).to(dtype)
    mask = torch.arange(S)[None, :] < torch.tensor([S, 131])[:, None]
    T = B * S
    valid = mask.reshape(T)
    keep = {}
    print(f"int8 block dtype={dtype} causal={causal}", flush=True)
    with torch.inference_mode():
        y = block_forward(blk, x.to(gpu), mask.to(gpu), causal, keep=keep)
    k = {n: t.cpu() for n, t in keep.items()}
    p = {n: t.detach().float().cpu() for n, t in blk.state_dict().items()}
    att = {n[len("attention."):]: t for n, t in p.items() if n.startswith("attention.")}
    pk, pf = OI.pack_block(att), OI.pack_ffn(p)
    xf = x.float().reshape(T, d)

    def ln_check(name, inp, w, b):
        r = compare_outputs(OA.layer_norm(inp, w, b).to(dtype).float(), k[name].float())
        print(f"  {name}:", r.summary(), flush=True)
        assert r.passed, r.summary()

    def quant_check(name, vals):
        q, s = OI.quant_rows(vals.float().numpy())
        np.testing.assert_array_equal(k[name + "_i8"].numpy(), q)
        np.testing.assert_array_equal(k[name + "_scale"].numpy(), s)
        return q, s

    ln_check("h", xf, p["norm1.weight"], p["norm1.bias"])
    hq, sh = quant_check("h", k["h"])
    qkv = OI.dequant(OI.int8_gemm(hq, pk["qkv_w"]), sh, pk["qkv_s"], pk["qkv_b"])
    assert torch.equal(k["qkv"], torch.from_numpy(qkv.astype(np.float16)))
    hd = d // H
    q5 = k["qkv"].float().view(B, S, 3, H, hd)
    q, kk, v = (q5[:, :, i].transpose(1, 2) for i in range(3))
    ctx = OA.attention_core(q, kk, v, hd ** -0.5, causal, mask).transpose(1, 2).reshape(T, d)
    r = compare_outputs(ctx, k["ctx"].reshape(T, d))
    print("  ctx vs fp32-math attention on the same qkv:", r.summary(), flush=True)
    assert r.passed, r.summary()
    cq, sc = quant_check("ctx", k["ctx"].reshape(T, d))
    o = _round(OI.dequant(OI.int8_gemm(cq, pk["out_w"]), sc, pk["out_s"], pk["out_b"]), dtype)
    x1 = (xf + o).to(dtype).float()
    x1[~valid] = xf[~valid]
    assert torch.equal(k["x1"].float(), x1)
    ln_check("h2", x1, p["norm2.weight"], p["norm2.bias"])
    h2q, sh2 = quant_check("h2", k["h2"])
    f = _round(OI.dequant(OI.int8_gemm(h2q, pf["f1_w"]), sh2, pf["f1_s"], pf["f1_b"]), dtype)
    exact = OB.gelu(f.double())
    ulp = _ulp(exact.float(), dtype).double()
    gd = (k["g"].double() - exact).abs()
    print(f"  gelu: max |d| / ulp {float((gd / ulp).max()):.3f}", flush=True)
    assert bool((gd <= ulp + 4e-7).all())
    gq, sg = quant_check("g", k["g"])
    o2 = _round(OI.dequant(OI.int8_gemm(gq, pf["f2_w"]), sg, pf["f2_s"], pf["f2_b"]), dtype)
    want = (x1 + o2).to(dtype).float()
    want[~valid] = 0
    assert torch.equal(y.reshape(T, d).float().cpu(), want)
    if dtype == torch.float32:
        # end to end vs the recipe: four requantisation points (h, ctx, h2, gelu output) turn
        # attention/LayerNorm rounding differences into int8 code moves; every stage above is
        # exact or within the predicate given our own intermediates, and at least
        # INT8_BLOCK_PASS_FLOOR of the output elements must pass the predicate end to end
        rec = OI.int8_transformer_block(x, p, H, mask, causal)["out"]
        r = compare_outputs(rec, y.cpu())
        frac = 1.0 - r.failed_elements / r.total_elements
        print(f"  end to end vs the int8 recipe: pass fraction {frac:.5f}:", r.summary(), flush=True)
        assert frac >= INT8_BLOCK_PASS_FLOOR, r.summary()
    flt = OB.transformer_block(x.float(), p, H, mask, causal)
    print("  reported: end to end vs the unquantised block:", compare_outputs(flt, y.cpu()).summary(),
          flush=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_int8_plugin_full_model_equals_transformer(gpu, dtype):
    """build(otb, config, int8=True, full_model=True) is the same computation as
    Transformer(config, int8=True); with fuse_block=True only the attention half runs on the
    kernels (Int8SelfAttention.forward_residual) and the FFN stays the reference's."""
    from tiktok_techjam_2026_track3_amd import Transformer, build
    cfg = OM.TransformerConfig(batch_size=2, seq_len=96, d_model=128, num_heads=2, ffn_dim=256,
                               num_layers=2, causal=True)
    torch.manual_seed(8)
    base = OM.BaselineTransformer(cfg)
    full = build(OM, cfg, int8=True, full_model=True)
    full.load_state_dict(base.state_dict(), strict=True)
    ours = Transformer(cfg, int8=True)
    ours.load_state_dict(base.state_dict(), strict=True)
    fused = build(OM, cfg, int8=True, fuse_block=True)
    fused.load_state_dict(base.state_dict(), strict=True)
    full, ours, fused = (m.to(device=gpu, dtype=dtype).eval() for m in (full, ours, fused))
    x = torch.randn(2, 96, 128, generator=torch.Generator().manual_seed(9)).to(dtype).to(gpu)
    mask = torch.ones(2, 96, dtype=torch.bool, device=gpu)
    mask[1, 70:] = False
    with torch.inference_mode():
        a, b = full(x, mask), ours(x, mask)
        assert torch.equal(a, b)
        l0 = fused.layers[0]
        x1 = l0.attention.forward_residual(x, l0.norm1, mask, True)
        assert torch.equal(x1, ours.layers[0].attention.forward_residual(x, ours.layers[0].norm1,
                                                                          mask, True))
        out = fused(x, mask)
    assert torch.isfinite(out).all() and torch.all(out[~mask] == 0)
