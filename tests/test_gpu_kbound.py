"""Key-norm bounds written by the QKV projection's epilogue (mi355_gemm_bias_kbound,
mi355_layernorm_gemm_bias_kbound) and read by the attention without its bound pass
(mi355_attn_fwd_kb with bounds_ready), and the block's policy that uses them.

Bars: the projection's outputs are bit for bit those of the plain projection; its bounds are bit
for bit those of the attention's own bound pass on the same K (sign bits of masked chunks
included); an attention call on projection-written bounds gives the bits of the same call with
the bound pass; the block's causal rows depend on no token after their 256-row tile (prefix runs
bit for bit), and its outputs pass the reference's predicate against the exact running max.
"""
import pytest
import torch

from oracle import attention as OA
from oracle.predicate import compare_outputs

pytestmark = pytest.mark.gpu


def _ops():
    from tiktok_techjam_2026_track3_amd import ops
    return ops


def _rand(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _bound_pass(gpu, q, k, v, causal, mask):
    """The bounds (as int32 bits) that mi355_attn_fwd_ws's bound pass writes for this K."""
    from tiktok_techjam_2026_track3_amd import _lib as L
    B, S, H, hd = q.shape
    n_kb = B * H * ((S + 255) // 256)
    ws = _ops().attention_workspace(B, S, S, H, hd, q.dtype, gpu)
    ws.fill_(0x7F)
    out = torch.empty_like(q)
    st = [L.i64_array((t.stride(0), t.stride(1), t.stride(2))) for t in (q, k, v, out)]
    rc = L.lib().mi355_attn_fwd_ws(L.dtype_code(q.dtype), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                   out.data_ptr(), B, H, S, S, hd, *st, hd ** -0.5, int(causal),
                                   None if mask is None else mask.data_ptr(),
                                   0 if mask is None else mask.stride(0),
                                   ws.data_ptr(), ws.numel(), None)
    L.check("mi355_attn_fwd_ws", rc)
    return ws[:4 * n_kb].view(torch.int32).cpu()


PAIRS = [(torch.float16, torch.float16), (torch.bfloat16, torch.float16),
         (torch.bfloat16, torch.bfloat16)]


@pytest.mark.parametrize("dt,odt", PAIRS)
@pytest.mark.parametrize("hd", [32, 64, 128])
@pytest.mark.parametrize("folded", [False, True])
@pytest.mark.parametrize("masked", [False, True])
def test_projection_bounds_are_the_bound_pass_bits(gpu, dt, odt, hd, folded, masked):
    """B 2, S 768, d 512 (K block = columns 512..1023 of the packed [T, 3d] output): the fused
    projection's output equals the plain projection's bit for bit, and its bounds equal the
    attention bound pass's, as bits (the key mask, when given, invalidates keys 300 and 767 of
    batch row 1: the sign bits of chunks 1 and 2 of its heads)."""
    ops = _ops()
    B, S, d = 2, 768, 512
    H = d // hd
    print(f"projection bounds {dt}->{odt} hd={hd} folded={folded} masked={masked}", flush=True)
    x = _rand((B * S, d), dt, 901, scale=2.0).to(gpu)
    w = _rand((3 * d, d), dt, 902, scale=d ** -0.5).to(gpu)
    b = _rand((3 * d,), torch.float32, 903, scale=0.1).to(gpu)
    mask = None
    if masked:
        m = torch.ones(B, S, dtype=torch.bool)
        m[1, 300] = False
        m[1, 767] = False
        mask = m.to(gpu)
    ws = ops.attention_workspace(B, S, S, H, hd, odt, gpu)
    ws.fill_(0x55)
    tgt = ops.KeyBoundTarget(ws, k_col0=d, heads=H, head_dim=hd, seq=S, key_valid=mask)
    if folded:
        colsum = w.float().sum(1)
        out = ops.layernorm_linear(x, w, colsum, b, 1e-5, out_dtype=odt, key_bounds=tgt)
        plain = ops.layernorm_linear(x, w, colsum, b, 1e-5, out_dtype=odt)
    else:
        out = ops.linear(x, w, b, out_dtype=odt, key_bounds=tgt)
        plain = ops.linear(x, w, b, out_dtype=odt)
    assert tgt.written
    assert torch.equal(out, plain)
    q, k, v = out.view(B, S, 3, H, hd).unbind(2)
    n_kb = B * H * (S // 256)
    fused = ws[:4 * n_kb].view(torch.int32).cpu()
    ref = _bound_pass(gpu, q, k, v, False, mask)
    assert torch.equal(fused, ref)
    signs = (fused < 0).view(B, H, S // 256)
    if masked:
        assert not signs[0].any() and not signs[1, :, 0].any() and signs[1, :, 1:].all()
    else:
        assert not signs.any()


@pytest.mark.parametrize("case", ["seq_not_256", "k_block_not_256", "fp32_input", "split_k"])
def test_projection_bounds_refused_shapes(gpu, case):
    """Shapes the fused epilogue cannot serve: nothing is written (``written`` False) and the
    projection is the plain one, bit for bit."""
    ops = _ops()
    B, S, d, hd, dt = 2, 768, 512, 64, torch.float16
    if case == "seq_not_256":
        S = 700
    elif case == "k_block_not_256":
        d = 384
    elif case == "fp32_input":
        dt = torch.float32
    elif case == "split_k":
        B, S, d = 1, 256, 256
    H = d // hd
    x = _rand((B * S, d), dt, 911).to(gpu)
    w = _rand((3 * d, d), dt, 912, scale=d ** -0.5).to(gpu)
    b = _rand((3 * d,), torch.float32, 913, scale=0.1).to(gpu)
    odt = torch.float16
    ws = ops.attention_workspace(B, S, S, H, hd, odt, gpu)
    ws.fill_(0x55)
    before = ws.clone()
    tgt = ops.KeyBoundTarget(ws, k_col0=d, heads=H, head_dim=hd, seq=S)
    out = ops.linear(x, w, b, out_dtype=odt, key_bounds=tgt)
    assert not tgt.written
    assert torch.equal(out, ops.linear(x, w, b, out_dtype=odt))
    assert torch.equal(ws, before)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("scale", [0.125, 1.0])
def test_attention_on_projection_bounds_same_bits(gpu, causal, masked, scale):
    """q, k, v from a fused fp16 projection (B 2, S 2048, d 512, head_dim 64): attention with
    bounds_ready gives the bits of the same call whose bound pass computes them, at causal sweep
    lengths 256 and 1024 (x at scale 0.125: the max-free sweep; at 1.0: the offset sweep), and
    passes the reference's predicate against the exact running max; with a key mask (batch row
    1's key 1500 invalid) the work-groups that see it run the key-masked path."""
    ops = _ops()
    B, S, d, hd = 2, 2048, 512, 64
    H = d // hd
    print(f"attention on projection bounds causal={causal} masked={masked} scale={scale}", flush=True)
    x = _rand((B * S, d), torch.float16, 921).to(gpu)
    w = _rand((3 * d, d), torch.float16, 922, scale=scale * d ** -0.5).to(gpu)
    b = torch.zeros(3 * d, device=gpu)
    mask = None
    if masked:
        m = torch.ones(B, S, dtype=torch.bool)
        m[1, 1500] = False
        mask = m.to(gpu)
    ws = ops.attention_workspace(B, S, S, H, hd, torch.float16, gpu)
    tgt = ops.KeyBoundTarget(ws, k_col0=d, heads=H, head_dim=hd, seq=S, key_valid=mask)
    qkv = ops.linear(x, w, b, out_dtype=torch.float16, key_bounds=tgt)
    assert tgt.written
    q, k, v = qkv.view(B, S, 3, H, hd).unbind(2)
    for gate in (256, 1024):
        ready = ops.attention(q, k, v, causal=causal, key_valid=mask, workspace=ws,
                              bounds_ready=True, causal_sweep_min_keys=gate)
        ws2 = ops.attention_workspace(B, S, S, H, hd, torch.float16, gpu)
        own = ops.attention(q, k, v, causal=causal, key_valid=mask, workspace=ws2,
                            bounds_ready=False, causal_sweep_min_keys=gate)
        assert torch.equal(ready, own)
    exact = ops.attention(q, k, v, causal=causal, key_valid=mask, key_bound=False)
    r = compare_outputs(exact.float().cpu(), ready.float().cpu())
    print("  vs exact running max:", r.summary(), flush=True)
    assert r.passed, r.summary()
    ref = OA.attention_core(*(t.cpu().double().transpose(1, 2) for t in (q, k, v)), hd ** -0.5,
                            causal, None if mask is None else mask.cpu()).transpose(1, 2)
    assert float((ready.double().cpu() - ref).abs().max()) < 2e-3


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_block_causal_bounds_policy_prefix_rows(gpu, dtype):
    """The attention half of a causal block (d 512, 8 heads of 64) at S 4096: causal calls from
    SelfAttention.causal_sweep_min_keys (2048) keys on take the projection's bounds and sweep
    their query tiles from that key range on. Output rows [0, P) equal a run on the first P
    tokens alone, bit for bit, for P = 2048 (bounds in both runs) and P = 1792 (none in the
    prefix run); the output passes the reference's predicate against the exact running max
    (key_bound False); a length that the projection cannot serve (S 4000: the bound pass) gives
    the same first 2048 rows as the fused run."""
    from tiktok_techjam_2026_track3_amd import SelfAttention
    B, S, d, H = 2, 4096, 512, 8
    print(f"block causal bounds policy dtype={dtype}", flush=True)
    torch.manual_seed(931)
    mod = SelfAttention(d, H).to(device=gpu, dtype=dtype).eval()
    mod.auto_graph = False
    norm = torch.nn.LayerNorm(d).to(device=gpu, dtype=dtype)
    x = _rand((B, S, d), dtype, 932).to(gpu)
    mask = torch.ones(B, S, dtype=torch.bool, device=gpu)
    with torch.inference_mode():
        full = mod.forward_residual(x, norm, mask, True)
        for P in (2048, 1792):
            pre = mod.forward_residual(x[:, :P].contiguous(), norm, mask[:, :P].contiguous(), True)
            assert torch.equal(pre, full[:, :P]), P
        odd = mod.forward_residual(x[:, :4000].contiguous(), norm, mask[:, :4000].contiguous(), True)
        assert torch.equal(odd[:, :2048], full[:, :2048])
        mod.key_bound = False
        exact = mod.forward_residual(x, norm, mask, True)
        mod.key_bound = None
    assert not torch.equal(full, exact)  # the sweeps ran
    r = compare_outputs(exact.float().cpu(), full.float().cpu())
    print("  vs exact running max:", r.summary(), flush=True)
    assert r.passed, r.summary()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
def test_block_padding_masks_with_projection_bounds(gpu, dtype, causal):
    """Padded rows (generate_random_case with padding_ratio > 0, torch_transformer_benchmark.py:
    254-271) at a shape whose QKV projection writes the bounds (B 2, S 2048, d 256, 4 heads):
    the chunks holding padded keys carry the sign bit, the work-groups that see them run the
    key-masked redo launch, the others the sweeps; the block passes the reference's predicate
    against the fp32 oracle and padded rows are zero."""
    from tiktok_techjam_2026_track3_amd import SelfAttention
    from tiktok_techjam_2026_track3_amd import workloads as W
    B, S, d, H = 2, 2048, 256, 4
    print(f"padding with projection bounds dtype={dtype} causal={causal}", flush=True)
    w = W.Workload("pad", B, S, d, H, dtype, causal, False, "normal_inv_d")
    params = W.round_params(W.make_params(w), dtype)
    x = W.make_input(w, 79)
    mask = torch.ones(B, S, dtype=torch.bool)
    mask[0, 1500:] = False   # row 0 padded from key 1500 on; row 1 unpadded
    x = x.masked_fill(~mask[..., None], 0)
    mod = SelfAttention(d, H)
    mod.load_state_dict(params)
    mod = mod.to(device=gpu, dtype=dtype)
    mod.auto_graph = False
    with torch.inference_mode():
        out = mod(x.to(gpu), mask.to(gpu), causal)
    ref = OA.self_attention(x.float(), {k: v.float() for k, v in params.items()}, H, mask, causal)
    r = compare_outputs(ref, out)
    print("  vs fp32 oracle:", r.summary(), flush=True)
    assert r.passed, r.summary()
    assert torch.all(out.cpu()[~mask] == 0)
