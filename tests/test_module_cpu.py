"""Module and plugin mechanics that need no GPU (mirrors the reference's SubmissionRuntimeTests,
Project/tools/tests/evidence_submission_test.py:729-811, minus the CPU compute route: this
build has no CPU path, so a CPU forward must raise instead of silently running torch)."""
import pytest
import torch

from oracle import model as OM
from tiktok_techjam_2026_track3_amd import (BaselineSelfAttention, Int8SelfAttention, SelfAttention,
                                            build, make_user_optimized_transformer, swap_attention,
                                            swap_blocks, swap_model)
from tiktok_techjam_2026_track3_amd import workloads as W


def test_same_attributes_and_state_dict_as_reference_module():
    torch.manual_seed(0)
    ref = OM.BaselineSelfAttention(64, 4)
    mine = SelfAttention(64, 4)
    assert list(ref.state_dict().keys()) == list(mine.state_dict().keys())
    for a in ("d_model", "num_heads", "head_dim", "scale"):
        assert getattr(ref, a) == getattr(mine, a)
    res = mine.load_state_dict(ref.state_dict(), strict=True)
    assert not res.missing_keys and not res.unexpected_keys
    assert BaselineSelfAttention is SelfAttention
    with pytest.raises(ValueError):
        SelfAttention(65, 4)


def test_cpu_forward_raises_instead_of_falling_back():
    mod = SelfAttention(32, 4)
    with pytest.raises(RuntimeError, match="no CPU path"):
        mod(torch.randn(1, 8, 32))
    with pytest.raises(ValueError):
        mod(torch.randn(1, 8, 16))


def test_graphed_forward_refuses_cpu_input():
    from tiktok_techjam_2026_track3_amd import GraphedForward
    mod = SelfAttention(64, 4)
    with pytest.raises(RuntimeError, match="GPU"):
        GraphedForward(mod, torch.zeros(1, 8, 64))


def test_graphed_forward_refuses_replay_once_the_weight_cache_changed():
    """The captured graph reads the module's packed weights by address: it holds the captured
    cache entry (so the tensors stay alive) and refuses to replay once the module dropped or
    rebuilt it -- a same-device .to() keeps every parameter's (data_ptr, version) but drops the
    cache. (The object is assembled by hand: capture itself needs a GPU.)"""
    from tiktok_techjam_2026_track3_amd import GraphedForward
    mod = SelfAttention(64, 4)
    gf = object.__new__(GraphedForward)
    gf.module, gf.norm, gf.causal = mod, None, False
    gf.static_x, gf.static_mask = torch.zeros(1, 8, 64), None
    mod.__dict__["_mi355_pack"] = (("stamp",), ("packed weights",))
    gf._stamp = gf._params_stamp()
    gf._cache = mod.__dict__.get("_mi355_pack")
    assert gf._cache_current()
    mod.to(torch.float32)                      # same device and dtype: parameters untouched
    assert gf._params_stamp() == gf._stamp     # the stamp alone would not notice
    assert not gf._cache_current()
    assert gf._cache == (("stamp",), ("packed weights",))   # the captured tensors stay referenced
    with pytest.raises(RuntimeError, match="changed since capture"):
        gf(torch.zeros(1, 8, 64))
    mod.__dict__["_mi355_pack"] = (("stamp",), ("rebuilt",))  # a rebuilt cache is refused too
    with pytest.raises(RuntimeError, match="changed since capture"):
        gf(torch.zeros(1, 8, 64))


def test_graphed_forward_refuses_replay_once_the_folded_norm_weights_changed():
    """The attention half's graph also reads the LayerNorm-folded QKV weights by address: a
    dropped or rebuilt fold (e.g. after norm1's parameters changed) refuses replay too."""
    from tiktok_techjam_2026_track3_amd import GraphedForward
    mod = SelfAttention(64, 4)
    norm = torch.nn.LayerNorm(64)
    gf = object.__new__(GraphedForward)
    gf.module, gf.norm, gf.causal = mod, norm, False
    gf.static_x, gf.static_mask = torch.zeros(1, 8, 64), None
    mod.__dict__["_mi355_pack"] = (("stamp",), ("packed weights",))
    mod.__dict__["_mi355_lnpack"] = (("ln stamp",), ("folded weights",))
    gf._stamp = gf._params_stamp()
    gf._cache = mod.__dict__.get("_mi355_pack")
    gf._ln_cache = mod.__dict__.get("_mi355_lnpack")
    assert gf._cache_current()
    mod.__dict__["_mi355_lnpack"] = (("ln stamp 2",), ("refolded",))
    assert not gf._cache_current()
    with pytest.raises(RuntimeError, match="changed since capture"):
        gf(torch.zeros(1, 8, 64))
    with torch.no_grad():
        norm.weight.add_(1.0)                  # the norm's parameters are in the stamp
    assert gf._params_stamp() != gf._stamp


def test_load_state_dict_and_apply_drop_derived_caches():
    mod = SelfAttention(32, 4)
    for key in ("_mi355_pack", "_mi355_lnpack"):
        mod.__dict__[key] = object()
        mod.load_state_dict(mod.state_dict(), strict=True)
        assert key not in mod.__dict__
        mod.__dict__[key] = object()
        mod.half()
        assert key not in mod.__dict__


def test_param_stamp_tracks_in_place_updates():
    mod = SelfAttention(32, 4)
    s1 = mod._param_stamp()
    with torch.no_grad():
        mod.q_proj.weight.mul_(2)
    assert mod._param_stamp() != s1


def test_core_dtype_policy():
    mod = SelfAttention(32, 4)
    assert mod.core_dtype(torch.float16) == torch.float16
    assert mod.core_dtype(torch.float32) == torch.float32
    assert mod.core_dtype(torch.bfloat16) == torch.float16


def test_plugin_build_and_swap_keep_state_dict_keys():
    cfg = OM.TransformerConfig(batch_size=2, seq_len=8, d_model=16, num_heads=4, ffn_dim=16,
                               num_layers=2, causal=True)
    torch.manual_seed(7)
    base = OM.BaselineTransformer(cfg)
    cand = build(OM, cfg)
    assert isinstance(cand, OM.UserOptimizedTransformer)
    assert all(type(l.attention) is SelfAttention for l in cand.layers)
    res = cand.load_state_dict(base.state_dict(), strict=True)
    assert not res.missing_keys and not res.unexpected_keys
    # class-swap idiom (k001_sdpa.py:55-61): parameters are the same objects afterwards
    params_before = [id(p) for p in base.parameters()]
    assert swap_attention(base, int8=True) == 2
    assert [id(p) for p in base.parameters()] == params_before
    assert all(type(l.attention) is Int8SelfAttention for l in base.layers)
    Uot = make_user_optimized_transformer(OM)
    m = Uot(cfg)
    assert issubclass(Uot, OM.BaselineTransformer)
    assert all(type(l.attention) is SelfAttention for l in m.layers)


def test_plugin_fuse_block_reclasses_blocks_only():
    from tiktok_techjam_2026_track3_amd.plugin import swap_blocks
    cfg = OM.TransformerConfig(batch_size=2, seq_len=8, d_model=16, num_heads=4, ffn_dim=16,
                               num_layers=3, causal=False)
    torch.manual_seed(9)
    base = OM.BaselineTransformer(cfg)
    cand = build(OM, cfg, fuse_block=True)
    assert all(isinstance(l, OM.BaselineTransformerBlock) for l in cand.layers)
    assert all(type(l).__name__ == "FusedBaselineTransformerBlock" for l in cand.layers)
    assert all(type(l.attention) is SelfAttention for l in cand.layers)
    assert len({type(l) for l in cand.layers}) == 1          # one derived class, reused
    res = cand.load_state_dict(base.state_dict(), strict=True)
    assert not res.missing_keys and not res.unexpected_keys
    assert swap_blocks(cand) == 3                             # idempotent: same classes again
    assert len({type(l) for l in cand.layers}) == 1
    # the int8 recipe swaps the same blocks with W8A8 attention (and keeps it on re-swaps)
    cand8 = build(OM, cfg, int8=True, fuse_block=True)
    assert all(type(l.attention) is Int8SelfAttention for l in cand8.layers)
    assert swap_blocks(cand8, int8=True) == 3
    assert all(type(l.attention) is Int8SelfAttention for l in cand8.layers)
    full8 = build(OM, cfg, int8=True, full_model=True)
    assert all(type(l.attention) is Int8SelfAttention for l in full8.layers)
    assert all(type(l).__name__.startswith("Kernel") for l in full8.layers)
    assert swap_model(full8) == 3                             # back to the 16-bit / fp32 attention
    assert all(type(l.attention) is SelfAttention for l in full8.layers)
    # no CPU route: the fused block's forward raises on CPU tensors
    with pytest.raises(Exception):
        cand(torch.randn(2, 8, 16), torch.ones(2, 8, dtype=torch.bool))
    with pytest.raises(RuntimeError, match="GPU"):
        Int8SelfAttention(16, 4).forward_residual(torch.randn(1, 8, 16), torch.nn.LayerNorm(16))


def test_workload_accounting():
    c2 = W.CONFIGS["C2"]
    f = c2.flops()
    assert f["qkv"] == 2 * 16384 * 1024 * 3072
    assert f["attn"] == 4 * 8 * 16 * 2048 ** 2 * 64
    c3 = W.CONFIGS["C3"]
    assert c3.flops()["attn"] == 4 * 4 * 32 * 8192 ** 2 * 64 / 2
    assert W.CONFIGS["C5"].flops()["attn"] == pytest.approx(655_360e9)
    p = W.make_params(W.CONFIGS["C1"])
    assert set(p) == {f"{n}.{t}" for n in W.PROJECTIONS for t in ("weight", "bias")}
    assert abs(p["q_proj.weight"].std().item() - 256 ** -0.5) < 0.01
    x1 = W.make_input(W.CONFIGS["C1"], 1234)
    x2 = W.make_input(W.CONFIGS["C1"], 1234)
    assert torch.equal(x1, x2) and x1.dtype == torch.float32
    # inputs and weights come from different streams
    assert not torch.allclose(x1[0, :256].reshape(-1)[:100], p["q_proj.weight"].reshape(-1)[:100] * 16)


def test_autograph_captures_form_no_reference_cycle():
    """A module's AutoGraph captures reference the module only weakly, so a dropped module frees
    its captured graphs at once (by reference counting) instead of leaving them to a later
    garbage collection, which could run while another graph records and would then free a graph
    in the middle of that capture. Checked on the CPU with a capture record built the way
    _Capture builds its references (its graph needs a GPU)."""
    import gc
    import weakref
    from tiktok_techjam_2026_track3_amd import graph as G
    m = SelfAttention(256, 4)
    m.__dict__["_mi355_pack"] = (torch.zeros(1),)
    cap = G._Capture.__new__(G._Capture)
    cap.caches = [(weakref.ref(mm), k, v) for mm, k, v in G._derived_caches(m)]
    cap.switch_mods = [weakref.ref(x) for x in G._switch_modules(m)]
    cap.switches = G._switch_values(G._alive(cap.switch_mods))
    assert cap.switches == G._switch_values(G._switch_modules(m))
    ag = G.AutoGraph()
    ag.entries[("signature",)] = {"cap": cap, "calls": 2, "failed": False}
    m.__dict__["_autograph"] = ag
    ref = weakref.ref(cap)
    was_on = gc.isenabled()
    gc.disable()
    try:
        del m, ag, cap
        assert ref() is None
    finally:
        if was_on:
            gc.enable()
    # a switch module that no longer exists gives a sentinel no recorded value equals
    assert G._switch_values([None]) == ((G._GONE,),)
