"""The evaluation harness's protocol checks on the eager module path and on graph replay.

Restates the candidate checks of Project/harness/candidate_worker.py:
  * input unchanged (:381-385): the forward must leave ``x`` and the mask bit-identical, and its
    output must pass the predicate against the fp32 oracle, per seed;
  * same-address fresh values (:431-451): five times, fresh random values are written into the
    SAME input buffer and the output must pass the predicate against the oracle of the new
    values -- an implementation that caches results by input address fails here;
  * the output is a fresh tensor, not an alias of an internal buffer that a later call
    overwrites (dispatcher_region.py:1335-1363).
"""
import pytest
import torch

from oracle import attention as OA
from oracle.predicate import compare_outputs
from tiktok_techjam_2026_track3_amd import workloads as W

pytestmark = pytest.mark.gpu

CASES = [("C2", 1, 256, True), ("C3", 1, 256, True), ("C1", 1, 128, True), ("C5", 1, 512, False)]


def _setup(gpu, name, batch, seq):
    from tiktok_techjam_2026_track3_amd import SelfAttention
    w = W.CONFIGS[name].scaled(batch, seq)
    params = W.round_params(W.make_params(w), w.dtype)
    mod = SelfAttention(w.d_model, w.heads)
    mod.load_state_dict(params)
    return w, params, mod.to(device=gpu, dtype=w.dtype)


def _oracle(w, params, x, mask):
    return OA.self_attention(x.float().cpu(), {k: v.float() for k, v in params.items()}, w.heads,
                             mask.cpu() if mask is not None else None, causal=w.causal)


@pytest.mark.parametrize("name,batch,seq,masked", CASES)
def test_inputs_unchanged_and_output_fresh(gpu, name, batch, seq, masked):
    w, params, mod = _setup(gpu, name, batch, seq)
    outs = []
    for seed in W.FIXED_SEEDS[:3]:
        x = W.make_input(w, seed, device="cuda")
        mask = torch.ones(w.batch, w.seq, dtype=torch.bool, device=gpu) if masked else None
        if masked:
            mask[:, w.seq - 7:] = False
        x_snap = x.clone()
        m_snap = None if mask is None else mask.clone()
        print(f"protocol {w.name} seed={seed}", flush=True)
        with torch.inference_mode():
            out = mod(x, mask, w.causal)
        torch.cuda.synchronize()
        assert torch.equal(x, x_snap), "the forward modified its input"
        if mask is not None:
            assert torch.equal(mask, m_snap), "the forward modified the mask"
        r = compare_outputs(_oracle(w, params, x, mask), out)
        assert r.passed, r.summary()
        outs.append((out, out.clone()))
    # earlier outputs were not overwritten by later calls (no shared output buffer)
    for out, snap in outs:
        assert torch.equal(out, snap)
    assert len({o.data_ptr() for o, _ in outs}) == len(outs)


@pytest.mark.parametrize("graphed", [False, True])
@pytest.mark.parametrize("name,batch,seq,masked", CASES[:3])
def test_same_address_fresh_values(gpu, name, batch, seq, masked, graphed):
    from tiktok_techjam_2026_track3_amd import GraphedForward
    w, params, mod = _setup(gpu, name, batch, seq)
    anti_x = W.make_input(w, W.BASE_SEED + 2_000_000, device="cuda")
    mask = torch.ones(w.batch, w.seq, dtype=torch.bool, device=gpu) if masked else None
    fwd = GraphedForward(mod, anti_x, mask, w.causal) if graphed else (
        lambda x, m: mod(x, m, w.causal))
    g = torch.Generator(device="cuda")
    prev = None
    for index in range(5):
        g.manual_seed(W.BASE_SEED + 3_000_000 + index)
        with torch.inference_mode():
            anti_x.copy_(torch.randn(anti_x.shape, generator=g, device=gpu).to(w.dtype))
            out = fwd(anti_x, mask)
        torch.cuda.synchronize()
        print(f"anti-cache {w.name} graphed={graphed} iteration {index}", flush=True)
        r = compare_outputs(_oracle(w, params, anti_x, mask), out)
        assert r.passed, r.summary()
        if prev is not None:
            assert not torch.equal(out, prev), "same output for fresh input values"
        prev = out.clone()


def _class_snapshot(mod):
    """Identity of every attribute of the official module's classes (methods, class attributes)."""
    out = {}
    for cname in ("BaselineSelfAttention", "BaselineTransformerBlock", "BaselineTransformer",
                  "UserOptimizedTransformer"):
        cls = getattr(mod, cname)
        out[cname] = (cls, cls.__mro__, {k: id(v) for k, v in vars(cls).items()})
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_baseline_invariance_probe(gpu, dtype):
    """The reference harness runs the official baseline on a probe input before any candidate
    is built and again after the candidate's trials, and requires bit-equal outputs
    (Project/harness/candidate_worker.py:352-360, 399-401): building candidates through every
    insertion point (build(otb, config) with each scope, make_user_optimized_transformer, the
    in-place swaps on a copy) and running them on the GPU must leave the official module's
    classes, the baseline's parameters and the baseline's output untouched. (The official
    module here is the oracle restatement, which runs on the CPU.)"""
    import copy
    from oracle import model as OM
    from tiktok_techjam_2026_track3_amd import build, make_user_optimized_transformer
    from tiktok_techjam_2026_track3_amd.plugin import swap_attention, swap_blocks, swap_model
    cfg = OM.TransformerConfig(batch_size=2, seq_len=256, d_model=256, num_heads=4, ffn_dim=512,
                               num_layers=2, causal=True)
    before = _class_snapshot(OM)
    torch.manual_seed(991)
    baseline = OM.BaselineTransformer(cfg).eval()
    state = {k: v.detach().clone() for k, v in baseline.state_dict().items()}
    g = torch.Generator().manual_seed(991_827_331)
    probe_x = torch.randn(2, 256, 256, generator=g)
    probe_mask = torch.ones(2, 256, dtype=torch.bool)
    probe_mask[1, 200:] = False
    with torch.inference_mode():
        probe_ref = baseline(probe_x, probe_mask).detach().clone()
    candidates = [build(OM, cfg), build(OM, cfg, fuse_block=True), build(OM, cfg, full_model=True),
                  make_user_optimized_transformer(OM)(cfg),
                  make_user_optimized_transformer(OM, full_model=True)(cfg)]
    for swap in (swap_attention, swap_blocks, swap_model):
        twin = copy.deepcopy(baseline)
        swap(twin)
        candidates.append(twin)
    x = torch.randn(2, 256, 256, generator=g).to(dtype).to(gpu)
    m = probe_mask.to(gpu)
    with torch.inference_mode():
        for cand in candidates:
            cand.load_state_dict(baseline.state_dict(), strict=True)
            cand = cand.to(device=gpu, dtype=dtype).eval()
            for _ in range(3):
                y = cand(x, m)
            assert torch.isfinite(y[m]).all()
        probe_now = baseline(probe_x, probe_mask)
    assert torch.equal(probe_now, probe_ref)
    assert _class_snapshot(OM) == before
    assert type(baseline) is OM.BaselineTransformer
    assert all(type(layer.attention) is OM.BaselineSelfAttention for layer in baseline.layers)
    for k, v in baseline.state_dict().items():
        assert torch.equal(v, state[k]), k
