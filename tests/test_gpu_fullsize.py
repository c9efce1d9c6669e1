"""GPU parity at the full measured shapes.

C2 is checked element by element against the dense CPU oracle, for the five fixed and two
random seeds. C3 and C5 are too large for a dense oracle (S x S scores of 34 GB / 10 TB), so sampled query rows (first, last, tile edges
and random) are checked against the streamed oracle (Project/tools/shape14_eval.py:201-236
semantics) computed from the full keys/values of their batch row; in addition, the full-size
call must equal per-batch-row calls bit for bit (the batch-decomposition property the
reference checks in shape14_eval.py:674-750), and every output must be finite; the other seeds
check sampled rows of one batch row each. C5's attention core on its own inputs (Q, K, V ~
N(0, 1) / 8) is checked on sampled rows for every seed. C4 is checked stage by stage on sampled
rows (bit-exact integer stages, predicate on attention) and end to end within the requantisation
bound.
"""
import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import int8 as OI
from oracle import streamed as OS
from oracle.predicate import compare_outputs
from tiktok_techjam_2026_track3_amd import workloads as W

import int8_requant
from test_gpu_block import INT8_E2E_PASS_FLOOR_FULL, SEEDS

pytestmark = pytest.mark.gpu

SEED = W.FIXED_SEEDS[0]


def _float_module(w, params, gpu):
    from tiktok_techjam_2026_track3_amd import SelfAttention
    mod = SelfAttention(w.d_model, w.heads)
    mod.load_state_dict(params)
    return mod.to(device=gpu, dtype=w.dtype)


def _sample_rows(S, n, seed):
    g = torch.Generator().manual_seed(seed)
    fixed = [0, 1, 63, 64, 127, 128, S // 2, S - 65, S - 64, S - 2, S - 1]
    rnd = torch.randint(0, S, (n,), generator=g).tolist()
    return torch.tensor(sorted(set(r for r in fixed + rnd if 0 <= r < S)))


def _sampled_oracle(x_row, pf, w, idx):
    """Oracle output rows ``idx`` of one batch row x_row [1, S, d] (fp32 math)."""
    S, d, H, hd = w.seq, w.d_model, w.heads, w.head_dim
    qkv = OA.qkv_projection(x_row.float(), pf).view(1, S, 3, H, hd)
    q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
    ctx = OS.streamed_attention_core(q[:, :, idx], k, v, hd ** -0.5, w.causal, q_index=idx)
    ctx = ctx.transpose(1, 2).reshape(1, len(idx), d)
    return torch.nn.functional.linear(ctx, pf["out_proj.weight"], pf["out_proj.bias"])


@pytest.mark.parametrize("seed", SEEDS)
def test_c2_full_dense(gpu, seed):
    w = W.CONFIGS["C2"]
    params = W.round_params(W.make_params(w), w.dtype)
    x = W.make_input(w, seed)
    mod = _float_module(w, params, gpu)
    print(f"C2 full B={w.batch} S={w.seq} seed={seed}", flush=True)
    with torch.inference_mode():
        out = mod(x.to(gpu), torch.ones(w.batch, w.seq, dtype=torch.bool, device=gpu), w.causal)
    torch.set_num_threads(16)
    ref = OA.self_attention(x.float(), {k: v.float() for k, v in params.items()}, w.heads)
    r = compare_outputs(ref, out)
    print(r.summary(), flush=True)
    assert r.passed, r.summary()


@pytest.mark.parametrize("name", ["C3", "C5"])
def test_long_sequence_sampled_rows_and_decomposition(gpu, name):
    w = W.CONFIGS[name]
    params = W.round_params(W.make_params(w), w.dtype)
    pf = {k: v.float() for k, v in params.items()}
    mod = _float_module(w, params, gpu)
    print(f"{name} full B={w.batch} S={w.seq} causal={w.causal}", flush=True)
    x = W.make_input(w, SEED, device="cuda")            # generated on the device (large)
    with torch.inference_mode():
        out = mod(x, None, w.causal)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        torch.set_num_threads(16)
        for b in (0, w.batch - 1):
            row = mod(x[b:b + 1].contiguous(), None, w.causal)
            assert torch.equal(row[0], out[b]), f"batch row {b} differs from the full call"
            idx = _sample_rows(w.seq, 24, 100 + b)
            ref = _sampled_oracle(x[b:b + 1].cpu(), pf, w, idx)
            r = compare_outputs(ref[0], out[b, idx])
            print(f"{name} batch {b}: {len(idx)} sampled rows: {r.summary()}", flush=True)
            assert r.passed, r.summary()


@pytest.mark.parametrize("seed", SEEDS[1:])
@pytest.mark.parametrize("name", ["C3", "C5"])
def test_long_sequence_more_seeds(gpu, name, seed):
    """The other fixed and random seeds at full size: sampled rows of one batch row (a different
    row per seed) against the streamed oracle."""
    w = W.CONFIGS[name]
    params = W.round_params(W.make_params(w), w.dtype)
    pf = {k: v.float() for k, v in params.items()}
    mod = _float_module(w, params, gpu)
    x = W.make_input(w, seed, device="cuda")
    b = seed % w.batch
    print(f"{name} full seed={seed} batch row {b}", flush=True)
    with torch.inference_mode():
        out = mod(x, None, w.causal)
    torch.cuda.synchronize()
    torch.set_num_threads(16)
    idx = _sample_rows(w.seq, 16, seed)
    ref = _sampled_oracle(x[b:b + 1].cpu(), pf, w, idx)
    r = compare_outputs(ref[0], out[b, idx])
    print(f"{name} seed {seed} batch {b}: {r.summary()}", flush=True)
    assert r.passed, r.summary()


@pytest.mark.parametrize("scale", ["c5", "unscaled"])
@pytest.mark.parametrize("seed", SEEDS)
def test_c5_attention_core_sampled_rows(gpu, seed, scale):
    """C5 as BASELINE states it: the streamed attention core on Q, K, V ~ N(0, 1) / sqrt(64)
    (B32 S100000 H8 x 64, fp16), sampled query rows of two batch rows against the chunk-wise
    oracle (shape14_eval.py:201-236) on the same rounded inputs; plus an unscaled N(0, 1)
    variant, whose softmax is far from uniform (numerical coverage, one seed)."""
    from tiktok_techjam_2026_track3_amd import ops
    if scale == "unscaled" and seed != SEED:
        pytest.skip("the unscaled variant runs on the first fixed seed only")
    w = W.CONFIGS["C5"]
    q, k, v = W.make_core_inputs(w, seed, device="cuda")
    if scale == "unscaled":
        q, k, v = ((t.float() * w.head_dim ** 0.5).to(w.dtype) for t in (q, k, v))
    print(f"C5 core seed={seed} scale={scale}", flush=True)
    with torch.inference_mode():
        out = ops.attention(q, k, v)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    torch.set_num_threads(16)
    for b in (seed % w.batch, (seed + 17) % w.batch):
        idx = _sample_rows(w.seq, 16, seed + b)
        qb, kb, vb = (t[b:b + 1].float().cpu().permute(0, 2, 1, 3) for t in (q, k, v))
        ref = OS.streamed_attention_core(qb[:, :, idx], kb, vb, w.head_dim ** -0.5, False,
                                         q_index=idx)
        r = compare_outputs(ref[0].transpose(0, 1), out[b, idx])
        print(f"C5 core batch {b}: {len(idx)} sampled rows: {r.summary()}", flush=True)
        assert r.passed, r.summary()


def test_c4_full_stagewise_sampled_rows(gpu):
    from tiktok_techjam_2026_track3_amd import Int8SelfAttention
    w = W.CONFIGS["C4"]
    params = W.make_params(w)
    mod = Int8SelfAttention(w.d_model, w.heads)
    mod.load_state_dict(params)
    mod = mod.to(gpu)
    T, d, H, hd, S = w.tokens, w.d_model, w.heads, w.head_dim, w.seq
    print(f"C4 full B={w.batch} S={S} d={d}", flush=True)
    x = W.make_input(w, SEED, device="cuda")
    keep = {}
    with torch.inference_mode():
        out = mod.run(x, None, w.causal, keep=keep)
        torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    pk = OI.pack_block(params)
    b = w.batch - 1
    idx = _sample_rows(S, 24, 7)
    rows = b * S + idx
    # activation quantisation + QKV (exact int32, fp32 dequant, fp16) on the sampled rows
    xs = x.reshape(T, d)[rows].float().cpu().numpy()
    xq, sx = OI.quant_rows(xs)
    np.testing.assert_array_equal(keep["x_i8"][rows].cpu().numpy(), xq)
    np.testing.assert_array_equal(keep["x_scale"][rows].cpu().numpy(), sx)
    acc = OI.int8_gemm(xq, pk["qkv_w"])
    qkv16 = OI.dequant(acc, sx, pk["qkv_s"], pk["qkv_b"]).astype(np.float16)
    np.testing.assert_array_equal(keep["qkv"][rows].cpu().numpy(), qkv16)
    # attention of the sampled queries from the full (GPU-produced, verified-format) K/V
    qkv_b = keep["qkv"].view(w.batch, S, 3, H, hd)[b].float().cpu()
    q = qkv_b[idx, 0].transpose(0, 1)[None]
    k = qkv_b[:, 1].transpose(0, 1)[None]
    v = qkv_b[:, 2].transpose(0, 1)[None]
    ctx_ref = OS.streamed_attention_core(q, k, v, hd ** -0.5, w.causal, q_index=idx)
    ctx = keep["ctx"].view(w.batch, S, H, hd)[b, idx].float().cpu()
    r = compare_outputs(ctx_ref[0].transpose(0, 1), ctx)
    print("C4 ctx sampled rows:", r.summary(), flush=True)
    assert r.passed, r.summary()
    # out projection from our context: bit-exact with the recipe
    y, _ = OI.int8_linear(keep["ctx"].view(T, d)[rows].float().cpu().numpy(),
                          pk["out_w"], pk["out_s"], pk["out_b"])
    assert torch.equal(out.reshape(T, d)[rows].cpu(), torch.from_numpy(y).to(torch.float16))
    # end to end against the recipe on the sampled rows: its own attention (probabilities
    # rounded to fp16, k008_int8_gemm.py:108, :218) on the same qkv, then its requantisation
    ctx_rec = OA.attention_core(q, k, v, hd ** -0.5, False, probs_dtype=torch.float16)
    ctx_rec = ctx_rec[0].transpose(0, 1).reshape(len(idx), d).to(torch.float16)
    frac, stats = int8_requant.check(keep["ctx"].view(T, d)[rows], ctx_rec, pk["out_w"],
                                     pk["out_s"], pk["out_b"], out.reshape(T, d)[rows])
    print("C4 end to end vs the recipe (sampled rows):", stats, flush=True)
    assert frac >= INT8_E2E_PASS_FLOOR_FULL, stats


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_official_shape14_attention_sampled_rows_to_the_end(gpu, dtype):
    """The attention of official shape 14 (B 32, S 100000, d 1024, 16 heads of 64, causal; the
    model's nn.Linear initialisation) on its real input size, as the model runs it (all-true
    mask, the library's default path at this length: key-norm bounds, the max-free and offset
    sweeps, redo launch). Sampled query rows up to position 99999 of two batch rows are checked
    stage by stage: the QKV projection against the oracle projection, the context against the
    chunk-wise oracle (Project/tools/shape14_eval.py:201-236) on the kernel's own rounded q/k/v,
    and the output against the oracle out projection of that context, by the reference's
    predicate."""
    from tiktok_techjam_2026_track3_amd import SelfAttention
    B, S, d, H = 32, 100000, 1024, 16
    hd = d // H
    torch.manual_seed(1414)
    mod = SelfAttention(d, H)
    params = {k: v.detach().clone() for k, v in mod.state_dict().items()}
    mod = mod.to(device=gpu, dtype=dtype)
    pf = {k: v.to(dtype).float() for k, v in params.items()}
    print(f"shape 14 attention dtype={dtype}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(14)
    x = torch.randn(B, S, d, device=gpu, generator=g).to(dtype)
    mask = torch.ones(B, S, dtype=torch.bool, device=gpu)
    keep = {}
    with torch.inference_mode():
        out = mod.run(x, mask, True, keep=keep)
        torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    torch.set_num_threads(16)
    fixed = [0, 255, 256, 2047, 2048, 32767, 32768, 65535, 65536, 99327, 99328, 99840, 99998, 99999]
    for b in (0, B - 1):
        g2 = torch.Generator().manual_seed(140 + b)
        idx = torch.tensor(sorted(set(fixed + torch.randint(0, S, (10,), generator=g2).tolist())))
        qkv_b = keep["qkv"].view(B, S, 3, H, hd)[b].float().cpu()
        ref_qkv = OA.qkv_projection(x[b, idx].float().cpu()[None], pf)[0]
        r = compare_outputs(ref_qkv, qkv_b[idx].reshape(len(idx), 3 * d))
        print(f"shape 14 batch {b}: qkv rows {r.summary()}", flush=True)
        assert r.passed, r.summary()
        q = qkv_b[idx, 0].transpose(0, 1)[None]
        k = qkv_b[:, 1].transpose(0, 1)[None]
        v = qkv_b[:, 2].transpose(0, 1)[None]
        ctx_ref = OS.streamed_attention_core(q, k, v, hd ** -0.5, True, q_index=idx)
        ctx = keep["ctx"].view(B, S, H, hd)[b, idx].float().cpu()
        r = compare_outputs(ctx_ref[0].transpose(0, 1), ctx)
        print(f"shape 14 batch {b}: context rows up to {int(idx.max())}: {r.summary()}",
              flush=True)
        assert r.passed, r.summary()
        y_ref = torch.nn.functional.linear(ctx.reshape(len(idx), d), pf["out_proj.weight"],
                                           pf["out_proj.bias"])
        r = compare_outputs(y_ref, out[b, idx].float().cpu())
        print(f"shape 14 batch {b}: output rows {r.summary()}", flush=True)
        assert r.passed, r.summary()
