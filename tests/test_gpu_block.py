"""GPU parity of the whole attention block against the CPU oracle (module API and plugin).

Tolerance: the benchmark's elementwise predicate ``finite AND (|d| <= 2e-3 OR |d| <= 2e-2*|ref|)``
(oracle.predicate) against fp32 math on the identically rounded inputs, over the five fixed
seeds 1234..1238 and two random seeds printed at collection. The int8 configuration is judged
against its quantised recipe (oracle.int8), whose integer stages are compared bit for bit.
Configurations run at reduced batch/sequence here (same d_model, heads, dtype, masking);
tests/test_gpu_fullsize.py covers the full shapes.
"""
import os
import random

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import int8 as OI
from oracle import model as OM
from oracle.predicate import compare_outputs
from tiktok_techjam_2026_track3_amd import workloads as W

import int8_requant

# fraction of the C4 attention-half output elements that must pass the predicate against the
# quantised recipe (the rest are bounded by their requantisation code moves, which is asserted
# per element). Measured 0.952-0.957 over seven seeds at the reduced shape (B1 S256 d4096):
# about 1% of the requantised context codes move by one step (a context value one fp16 ulp from
# the recipe's, next to a rounding boundary), every row has some, and each moved code shifts its
# row's outputs by up to s_ctx*|w|*s_w. The floor sits just under that spread, as a guard
# against a context that drifts further from the recipe's.
INT8_E2E_PASS_FLOOR = 0.945
# the same at the full C4 size (sampled rows) and on the committed golden case, where far fewer
# codes sit next to a boundary: measured 0.9998 and 1.0
INT8_E2E_PASS_FLOOR_FULL = 0.999

pytestmark = pytest.mark.gpu

_rng = random.Random(int.from_bytes(os.urandom(4), "little"))
RANDOM_SEEDS = tuple(_rng.randrange(2 ** 31) for _ in range(2))
print(f"random seeds for this run: {RANDOM_SEEDS}", flush=True)
SEEDS = W.FIXED_SEEDS + RANDOM_SEEDS

REDUCED = {"C1": (1, 128), "C2": (1, 1024), "C3": (1, 1024), "C4": (1, 256), "C5": (2, 2048)}


def _module(w, params, gpu):
    from tiktok_techjam_2026_track3_amd import Int8SelfAttention, SelfAttention
    cls = Int8SelfAttention if w.int8 else SelfAttention
    mod = cls(w.d_model, w.heads)
    mod.load_state_dict(params, strict=True)
    # int8 weights are quantised from the fp32 master weights; float configs hold w.dtype weights
    return mod.to(gpu) if w.int8 else mod.to(device=gpu, dtype=w.dtype)


def _float_case(name, seed, gpu, mask=True):
    w = W.CONFIGS[name].scaled(*REDUCED[name])
    params = W.round_params(W.make_params(w), w.dtype)
    x = W.make_input(w, seed)
    mod = _module(w, params, gpu)
    valid = torch.ones(w.batch, w.seq, dtype=torch.bool, device=gpu) if mask else None
    print(f"block {w.name} seed={seed} dtype={w.dtype} causal={w.causal}", flush=True)
    with torch.inference_mode():
        out = mod(x.to(gpu), valid, w.causal)
    assert out.dtype == w.dtype and out.shape == x.shape
    ref = OA.self_attention(x.float(), {k: v.float() for k, v in params.items()}, w.heads,
                            causal=w.causal)
    return compare_outputs(ref, out)


@pytest.mark.parametrize("seed", SEEDS)
@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C5"])
def test_block_matches_fp32_oracle(gpu, name, seed):
    r = _float_case(name, seed, gpu)
    print(r.summary(), flush=True)
    assert r.passed, r.summary()


@pytest.mark.parametrize("seed", SEEDS)
def test_int8_block_stages_match_quantised_recipe(gpu, seed):
    """C4 (W8A8). Every integer or rounded stage is compared bit for bit with the recipe
    (k008_int8_gemm.py:148-223): activation quantisation, the fp16 QKV after exact int32
    accumulation and dequantisation, and the out projection of the context. The attention stage
    (fp16 probabilities, fp32 accumulation) is held to the predicate against the recipe's own
    attention on the same fp16 qkv. End to end, the recipe re-quantises the context per token,
    so a context value next to a quantisation boundary can round to the neighbouring code:
    every code may move by at most one step, every output element must stay within the bound
    those code moves imply (tests/int8_requant.py), and at least INT8_E2E_PASS_FLOOR of the
    elements must pass the predicate against the recipe.
    """
    from tiktok_techjam_2026_track3_amd import Int8SelfAttention
    w = W.CONFIGS["C4"].scaled(*REDUCED["C4"])
    params = W.make_params(w)                      # fp32 master weights
    x = W.make_input(w, seed)                      # fp16 activations
    mod = _module(w, params, gpu)
    assert isinstance(mod, Int8SelfAttention)
    keep = {}
    print(f"int8 block {w.name} seed={seed}", flush=True)
    with torch.inference_mode():
        out = mod.run(x.to(gpu), None, w.causal, keep=keep)
    want = OI.int8_self_attention(x, params, w.heads, w.causal)
    T, d = w.tokens, w.d_model
    pk = OI.pack_block(params)
    xq, sx = OI.quant_rows(x.float().reshape(T, d).numpy())
    np.testing.assert_array_equal(keep["x_i8"].cpu().numpy(), xq)
    np.testing.assert_array_equal(keep["x_scale"].cpu().numpy(), sx)
    assert torch.equal(keep["qkv"].cpu(), want["qkv16"].reshape(T, 3 * d))
    r_ctx = compare_outputs(want["ctx16"].float(), keep["ctx"].reshape(T, d))
    print("ctx vs fp32-math attention on the same qkv:", r_ctx.summary(), flush=True)
    assert r_ctx.passed, r_ctx.summary()
    cq, sc = OI.quant_rows(keep["ctx"].reshape(T, d).float().cpu().numpy())
    np.testing.assert_array_equal(keep["ctx_i8"].cpu().numpy(), cq)
    np.testing.assert_array_equal(keep["ctx_scale"].cpu().numpy(), sc)
    y_from_ours, _ = OI.int8_linear(keep["ctx"].reshape(T, d).float().cpu().numpy(),
                                    pk["out_w"], pk["out_s"], pk["out_b"])
    assert torch.equal(out.reshape(T, d).cpu(), torch.from_numpy(y_from_ours).to(torch.float16))
    frac, stats = int8_requant.check(keep["ctx"].reshape(T, d), want["ctx16"], pk["out_w"],
                                     pk["out_s"], pk["out_b"], out.reshape(T, d))
    print("end to end vs quantised recipe:", stats, flush=True)
    assert frac >= INT8_E2E_PASS_FLOOR, stats
    ref32 = OA.self_attention(x.float(), params, w.heads, causal=w.causal)
    print("reported: end to end vs unquantised fp32 block:", compare_outputs(ref32, out).summary(),
          flush=True)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("causal", [False, True])
def test_block_padding_masks(gpu, dtype, causal):
    """generate_random_case with padding_ratio > 0 (torch_transformer_benchmark.py:254-271)."""
    from tiktok_techjam_2026_track3_amd import SelfAttention
    B, S, d, H = 4, 300, 256, 4
    w = W.Workload("pad", B, S, d, H, dtype, causal, False, "normal_inv_d")
    params = W.round_params(W.make_params(w), dtype)
    x = W.make_input(w, 77)
    g = torch.Generator().manual_seed(78)
    lengths = torch.randint(int(round(S * 0.5)), S + 1, (B,), generator=g)
    mask = torch.arange(S)[None, :] < lengths[:, None]
    x = x.masked_fill(~mask[..., None], 0)
    mod = SelfAttention(d, H)
    mod.load_state_dict(params)
    mod = mod.to(device=gpu, dtype=dtype)
    with torch.inference_mode():
        out = mod(x.to(gpu), mask.to(gpu), causal)
    ref = OA.self_attention(x.float(), {k: v.float() for k, v in params.items()}, H, mask, causal)
    r = compare_outputs(ref, out)
    print(r.summary(), flush=True)
    assert r.passed, r.summary()
    assert torch.all(out.cpu()[~mask] == 0)


def test_weight_updates_invalidate_packed_caches(gpu):
    from tiktok_techjam_2026_track3_amd import SelfAttention
    w = W.CONFIGS["C2"].scaled(1, 128)
    p1 = W.round_params(W.make_params(w, seed=1), w.dtype)
    p2 = W.round_params(W.make_params(w, seed=2), w.dtype)
    x = W.make_input(w, 5)
    mod = SelfAttention(w.d_model, w.heads).to(device=gpu, dtype=w.dtype)
    mod.load_state_dict(p1)
    with torch.inference_mode():
        o1 = mod(x.to(gpu)).cpu()
        mod.load_state_dict(p2)                  # strict copy, the harness's weight transfer
        o2 = mod(x.to(gpu)).cpu()
        with torch.no_grad():
            mod.out_proj.bias.add_(1.0)          # in-place update bumps the version counter
        o3 = mod(x.to(gpu)).cpu()
    ref2 = OA.self_attention(x.float(), {k: v.float() for k, v in p2.items()}, w.heads)
    assert compare_outputs(ref2, o2).passed
    assert not torch.equal(o1, o2)
    assert compare_outputs(ref2 + 1.0, o3).passed


def test_cuda_graph_replay_matches_eager(gpu):
    """The forward allocates through torch only and never syncs: it can be graph-captured."""
    from tiktok_techjam_2026_track3_amd import SelfAttention
    w = W.CONFIGS["C2"].scaled(1, 256)
    params = W.round_params(W.make_params(w), w.dtype)
    mod = SelfAttention(w.d_model, w.heads)
    mod.load_state_dict(params)
    mod = mod.to(device=gpu, dtype=w.dtype)
    static_x = W.make_input(w, 9).to(gpu)
    with torch.inference_mode():
        mod(static_x)                            # builds the packed-weight cache
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            mod(static_x)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_out = mod(static_x)
        for seed in (10, 11, 12):
            x = W.make_input(w, seed).to(gpu)
            static_x.copy_(x)
            graph.replay()
            eager = mod(x)
            torch.cuda.synchronize()
            assert torch.equal(static_out, eager)


def test_plugin_build_matches_oracle_transformer(gpu):
    """build(otb, config) on the oracle's restatement of the official module."""
    from tiktok_techjam_2026_track3_amd import SelfAttention, build
    cfg = OM.TransformerConfig(batch_size=2, seq_len=256, d_model=256, num_heads=4, ffn_dim=512,
                               num_layers=2, causal=True)
    torch.manual_seed(1234)
    baseline = OM.BaselineTransformer(cfg)
    cand = build(OM, cfg)
    incompatible = cand.load_state_dict(baseline.state_dict(), strict=True)
    assert not incompatible.missing_keys and not incompatible.unexpected_keys
    assert all(isinstance(l.attention, SelfAttention) for l in cand.layers)
    cand = cand.to(gpu).eval()
    x = torch.randn(2, 256, 256, generator=torch.Generator().manual_seed(1235))
    mask = torch.ones(2, 256, dtype=torch.bool)
    with torch.inference_mode():
        ref = baseline.eval()(x, mask)
        out = cand(x.to(gpu), mask.to(gpu))
    r = compare_outputs(ref, out)
    print(r.summary(), flush=True)
    assert r.passed, r.summary()


@pytest.mark.parametrize("name,masked,half", [("C1", True, False), ("C2", False, False),
                                              ("C3", True, True)])
def test_graphed_forward_replays_match_eager(gpu, name, masked, half):
    """GraphedForward (whole-forward capture): every replay equals the eager forward bit for bit,
    with unrelated eager work and synchronisations between replays; a parameter update after
    capture is refused."""
    from tiktok_techjam_2026_track3_amd import GraphedForward, SelfAttention
    w = W.CONFIGS[name].scaled(1, 128 if name == "C1" else 256)
    params = W.round_params(W.make_params(w), w.dtype)
    mod = SelfAttention(w.d_model, w.heads)
    mod.load_state_dict(params)
    mod = mod.to(device=gpu, dtype=w.dtype)
    norm = torch.nn.LayerNorm(w.d_model).to(device=gpu, dtype=w.dtype) if half else None
    mask = torch.ones(w.batch, w.seq, dtype=torch.bool, device=gpu) if masked else None
    if masked:
        mask[:, w.seq - 5:] = False
    gf = GraphedForward(mod, W.make_input(w, 40).to(gpu), mask, w.causal, norm=norm)
    with torch.inference_mode():
        for seed in (41, 42, 43):
            x = W.make_input(w, seed).to(gpu)
            got = gf(x, mask)
            noise = torch.randn(257, 129, device=gpu).sum()   # eager work between replays
            torch.cuda.synchronize()
            want = mod.forward_residual(x, norm, mask, w.causal) if half else mod(x, mask, w.causal)
            torch.cuda.synchronize()
            assert torch.isfinite(noise)
            assert torch.equal(got, want), f"replay for seed {seed} differs from eager"
        with torch.no_grad():
            mod.out_proj.bias.add_(1.0)
        with pytest.raises(RuntimeError):
            gf(x, mask)
