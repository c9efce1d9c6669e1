"""Graph replay inside the modules' forward (graph.AutoGraph) at launch-bound shapes: every call
must give the eager path's bits, whatever the caller does between calls (the reference's
protocol: fresh inputs at the same address, in-place updates, weight reloads, output ownership;
Project/harness/candidate_worker.py:381-385, 431-451)."""
import copy

import pytest
import torch

from oracle import model as OM

pytestmark = pytest.mark.gpu


def _attn(gpu, dtype, d=256, heads=4, seed=0):
    from tiktok_techjam_2026_track3_amd import SelfAttention
    torch.manual_seed(seed)
    return SelfAttention(d, heads).to(device=gpu, dtype=dtype).eval()


def _x(gpu, dtype, B=1, S=128, d=256, seed=1):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(B, S, d, generator=g).to(dtype).to(gpu)


def _captured(mod):
    ag = mod.__dict__.get("_autograph")
    return 0 if ag is None else sum(e["cap"] is not None for e in ag.entries.values())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("masked", [False, True])
def test_forward_replay_equals_eager(gpu, dtype, causal, masked):
    mod = _attn(gpu, dtype)
    x = _x(gpu, dtype)
    mask = None
    if masked:
        mask = torch.ones(1, 128, dtype=torch.bool, device=gpu)
        mask[0, 100:] = False
    with torch.inference_mode():
        want = mod.run(x, mask, causal)
        outs = [mod(x, mask, causal) for _ in range(4)]
    assert _captured(mod) == 1
    for o in outs:
        assert torch.equal(o, want)
    assert all(outs[i].data_ptr() != outs[j].data_ptr() for i in range(4) for j in range(i))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal,S", [(False, 512), (True, 2048)])
@pytest.mark.parametrize("masked", [False, True])
def test_forward_replay_with_projection_bounds_equals_eager(gpu, dtype, causal, S, masked):
    """Shapes where the QKV projection writes the attention's key-norm bounds (S and d multiples
    of 256; causal from SelfAttention.causal_sweep_min_keys keys on): the captured forward (the
    projection's bound epilogue, the sweep launch and the redo launch, with their workspace
    allocated inside the capture) gives the eager bits on every replay, with eager work between
    replays; with a key mask, the work-groups that see its invalid keys go to the key-masked
    redo launch in both."""
    mod = _attn(gpu, dtype)
    x = _x(gpu, dtype, S=S)
    mask = None
    if masked:
        mask = torch.ones(1, S, dtype=torch.bool, device=gpu)
        mask[0, S - 200] = False
    with torch.inference_mode():
        want = mod.run(x, mask, causal)
        outs = []
        for _ in range(4):
            outs.append(mod(x, mask, causal))
            mod.run(x, mask, not causal)  # eager work between the replays
    assert _captured(mod) == 1
    for o in outs:
        assert torch.equal(o, want)


def test_forward_sees_in_place_updates_and_new_tensors(gpu):
    dtype = torch.float16
    mod = _attn(gpu, dtype)
    x = _x(gpu, dtype)
    mask = torch.ones(1, 128, dtype=torch.bool, device=gpu)
    with torch.inference_mode():
        for _ in range(3):
            mod(x, mask)
        assert _captured(mod) == 1
        # in place, through the tensor and through a view (both bump the version counter)
        x.copy_(_x(gpu, dtype, seed=2))
        assert torch.equal(mod(x, mask), mod.run(x, mask))
        x.view(-1)[:1000].mul_(-1.0)
        assert torch.equal(mod(x, mask), mod.run(x, mask))
        mask[0, 64:] = False
        assert torch.equal(mod(x, mask), mod.run(x, mask))
        # a fresh tensor (possibly at a recycled address) each call
        for s in range(3, 6):
            y = _x(gpu, dtype, seed=s)
            assert torch.equal(mod(y, mask), mod.run(y, mask))
        # an inference tensor (no version counter) updated in place between calls
        z = _x(gpu, dtype, seed=6).clone()
        assert z.is_inference()
        for s in range(7, 10):
            mod(z, mask)
            z.copy_(_x(gpu, dtype, seed=s))
            assert torch.equal(mod(z, mask), mod.run(z, mask))


def test_forward_sees_switch_changes(gpu):
    """A graph captured with one set of module switches is recorded again when one changes: an
    fp32 model's core dtype switched to fp32 (the vector-ALU attention instead of the fp16
    matrix-core one) after capture gives the eager fp32-core bits, and the switch back the
    fp16-core bits again; the same for a transformer's LayerNorm eps."""
    from tiktok_techjam_2026_track3_amd import Transformer
    dtype = torch.float32
    mod = _attn(gpu, dtype)
    x = _x(gpu, dtype)
    with torch.inference_mode():
        half_core = mod.run(x)
        for _ in range(3):
            assert torch.equal(mod(x), half_core)
        assert _captured(mod) == 1
        mod.fp32_core_dtype = torch.float32
        full_core = mod.run(x)
        assert not torch.equal(full_core, half_core)
        for _ in range(3):
            assert torch.equal(mod(x), full_core)
        del mod.fp32_core_dtype                       # back to the class default
        for _ in range(3):
            assert torch.equal(mod(x), half_core)
    cfg = OM.TransformerConfig(batch_size=1, seq_len=64, d_model=128, num_heads=4, ffn_dim=256,
                               num_layers=2, causal=True)
    torch.manual_seed(5)
    model = Transformer(cfg).to(device=gpu, dtype=torch.float16).eval()
    y = _x(gpu, torch.float16, S=64, d=128, seed=3)
    with torch.inference_mode():
        for _ in range(3):
            a = model(y)
        model.layers[1].norm2.eps = 0.5
        model.auto_graph = False
        want = model(y)
        model.auto_graph = True
        assert not torch.equal(a, want)
        for _ in range(3):
            assert torch.equal(model(y), want)


def test_forward_outputs_are_owned_by_the_caller(gpu):
    dtype = torch.float16
    mod = _attn(gpu, dtype)
    xs = [_x(gpu, dtype, seed=s) for s in range(4)]
    with torch.inference_mode():
        want = [mod.run(x) for x in xs]
        got = [mod(x) for x in xs]
    for g, w in zip(got, want):
        assert torch.equal(g, w)


def test_forward_follows_weight_changes(gpu):
    dtype = torch.float16
    mod = _attn(gpu, dtype)
    other = _attn(gpu, dtype, seed=7)
    x = _x(gpu, dtype)
    with torch.inference_mode():
        for _ in range(3):
            mod(x)
        mod.load_state_dict(other.state_dict())
        assert torch.equal(mod(x), other.run(x))
        mod.out_proj.bias.add_(0.25)
        assert torch.equal(mod(x), mod.run(x))
    # a same-device same-dtype .to() drops the derived weights without moving the parameters
    mod = mod.to(device=gpu, dtype=dtype)
    with torch.inference_mode():
        for _ in range(3):
            assert torch.equal(mod(x), mod.run(x))
    # a parameter replaced by assignment (a new object, registered anew)
    mod.v_proj.weight = torch.nn.Parameter(other.v_proj.weight.detach() * 0.5)
    with torch.inference_mode():
        for _ in range(3):
            assert torch.equal(mod(x), mod.run(x))
    # the module's class swapped after capture (the reference's class-swap idiom)
    from tiktok_techjam_2026_track3_amd import SelfAttention

    class Swapped(SelfAttention):
        def run(self, x, valid_token_mask=None, causal=False, keep=None, marks=None):
            return super().run(x, valid_token_mask, causal, keep, marks) * 2
    with torch.inference_mode():
        mod.__class__ = Swapped
        for _ in range(3):
            assert torch.equal(mod(x), mod.run(x))


def test_forward_signatures_alternate(gpu):
    dtype = torch.float32
    mod = _attn(gpu, dtype)
    a, b = _x(gpu, dtype), _x(gpu, dtype, B=2, S=64, seed=3)
    with torch.inference_mode():
        for _ in range(3):
            for x in (a, b):
                for causal in (False, True):
                    assert torch.equal(mod(x, None, causal), mod.run(x, None, causal))
    assert _captured(mod) == 4


def test_large_inputs_and_outer_capture_stay_eager(gpu):
    dtype = torch.float16
    mod = _attn(gpu, dtype)
    big = _x(gpu, dtype, B=8, S=4096)            # 2^23 elements: above the replay limit
    x = _x(gpu, dtype)
    with torch.inference_mode():
        for _ in range(3):
            assert torch.equal(mod(big), mod.run(big))
        assert _captured(mod) == 0
        # inside the caller's own capture the forward records its kernels eagerly
        static_x = x.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            mod(static_x)
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = mod(static_x)
        for s in (4, 5):
            static_x.copy_(_x(gpu, dtype, seed=s))
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, mod.run(static_x))
    mod2 = copy.deepcopy(mod)                      # copies start without captures
    assert _captured(mod2) == 0
    with torch.inference_mode():
        assert torch.equal(mod2(x), mod.run(x))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_transformer_forward_replay_equals_eager(gpu, dtype):
    """The whole model at official shape 2 (B1 S128 d128, 4 layers): forward replays its graph
    from the second call, bit for bit the eager model, also after a weight reload."""
    from tiktok_techjam_2026_track3_amd import Transformer
    cfg = OM.TransformerConfig(batch_size=1, seq_len=128, d_model=128, num_heads=4, ffn_dim=128,
                               num_layers=4, causal=True)
    torch.manual_seed(11)
    model = Transformer(cfg).to(device=gpu, dtype=dtype).eval()
    x = _x(gpu, dtype, d=128)
    mask = torch.ones(1, 128, dtype=torch.bool, device=gpu)
    with torch.inference_mode():
        model.auto_graph = False
        want = model(x, mask)
        model.auto_graph = True
        for _ in range(4):
            assert torch.equal(model(x, mask), want)
        assert _captured(model) == 1
    torch.manual_seed(12)
    fresh = Transformer(cfg).to(device=gpu, dtype=dtype).eval()
    fresh.auto_graph = False
    with torch.inference_mode():
        model.load_state_dict(fresh.state_dict())
        assert torch.equal(model(x, mask), fresh(x, mask))
