"""Pins of the CPU oracle (no GPU): closed forms, invariances, brute force and hand cases.

The reference holds no golden vectors for this path, so every oracle function is pinned here
against mathematics that a plausible mistake (dropped scale, wrong mask diagonal, transposed
operand, wrong rounding mode, wrong clamp order) breaks. A few tests plant such mistakes in a
copy of the oracle computation to show the pins discriminate.
"""
import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import int8 as OI
from oracle import predicate as OP
from oracle import streamed as OS


def _params(d, seed=0, scale=0.3):
    g = torch.Generator().manual_seed(seed)
    p = {}
    for n in OA.PARAM_NAMES:
        p[f"{n}.weight"] = torch.randn(d, d, generator=g) * scale
        p[f"{n}.bias"] = torch.randn(d, generator=g) * 0.1
    return p


def _qkv(B, H, S, D, seed=0, Sk=None):
    g = torch.Generator().manual_seed(seed)
    Sk = Sk or S
    return (torch.randn(B, H, S, D, generator=g), torch.randn(B, H, Sk, D, generator=g),
            torch.randn(B, H, Sk, D, generator=g))


# ------------------------------------------------------------------ dense vs fp64 brute force
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("masked", [False, True])
def test_block_matches_bruteforce(causal, masked):
    B, S, d, H = 2, 7, 16, 4
    p = _params(d)
    x = torch.randn(B, S, d, generator=torch.Generator().manual_seed(1))
    mask = None
    if masked:
        mask = torch.ones(B, S, dtype=torch.bool)
        mask[1, 5:] = False
    got = OA.self_attention(x, p, H, mask, causal)
    want = OA.self_attention_bruteforce(x.numpy(), {k: v.numpy() for k, v in p.items()}, H, causal,
                                        None if mask is None else mask.numpy())
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-5, atol=1e-5)


def test_core_rectangular_matches_bruteforce():
    q, k, v = _qkv(1, 2, 5, 8, Sk=9)
    got = OA.attention_core(q, k, v, 0.35)
    want = OA.attention_core_bruteforce(q.numpy(), k.numpy(), v.numpy(), 0.35)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("mistake", ["scale", "diagonal", "transpose_v"])
def test_planted_mistakes_fail_the_bruteforce_pin(mistake):
    q, k, v = _qkv(1, 1, 6, 8, seed=3)
    want = OA.attention_core_bruteforce(q.numpy(), k.numpy(), v.numpy(), 8 ** -0.5, causal=True)
    scores = q @ k.transpose(-2, -1) * (8 ** -0.5 if mistake != "scale" else 1.0)
    diag = 0 if mistake == "diagonal" else 1
    scores = scores.masked_fill(torch.ones(6, 6, dtype=torch.bool).triu(diag), float("-inf"))
    probs = torch.softmax(scores, -1)
    if mistake == "diagonal":
        probs = torch.nan_to_num(probs)
    vv = v.transpose(-2, -1)[..., :6, :6] if mistake == "transpose_v" else v
    bad = (probs @ vv[..., :6, :]) if mistake != "transpose_v" else probs @ vv
    assert not np.allclose(bad.numpy()[..., : want.shape[-1]], want[..., : bad.shape[-1]], atol=1e-3)


# ------------------------------------------------------------------------- closed forms
def test_single_key_returns_its_value():
    q, k, v = _qkv(2, 3, 4, 8, Sk=1)
    out = OA.attention_core(q, k, v, 0.5)
    torch.testing.assert_close(out, v.expand(2, 3, 4, 8), rtol=0, atol=1e-7)


def test_equal_scores_average_values():
    _, k, v = _qkv(1, 2, 6, 8)
    q = torch.zeros(1, 2, 6, 8)
    out = OA.attention_core(q, k, v, 1.0)
    torch.testing.assert_close(out, v.mean(dim=2, keepdim=True).expand_as(out), rtol=1e-6, atol=1e-6)
    out_c = OA.attention_core(q, k, v, 1.0, causal=True)
    prefix_means = torch.cumsum(v, dim=2) / torch.arange(1, 7).view(1, 1, 6, 1)
    torch.testing.assert_close(out_c, prefix_means, rtol=1e-6, atol=1e-6)


def test_causal_first_row_is_first_value_and_constant_v():
    q, k, v = _qkv(1, 2, 5, 8)
    out = OA.attention_core(q, k, v, 0.4, causal=True)
    torch.testing.assert_close(out[:, :, 0], v[:, :, 0], rtol=0, atol=1e-7)
    vc = torch.full_like(v, 1.75)
    torch.testing.assert_close(OA.attention_core(q, k, vc, 0.4), torch.full_like(q, 1.75))


def test_key_permutation_and_score_shift_invariance():
    q, k, v = _qkv(1, 2, 5, 8, Sk=7)
    base = OA.attention_core(q, k, v, 0.3)
    perm = torch.randperm(7, generator=torch.Generator().manual_seed(5))
    torch.testing.assert_close(OA.attention_core(q, k[:, :, perm], v[:, :, perm], 0.3), base)
    # scores + c: append a constant feature to q and k
    q1 = torch.cat([q, torch.ones(1, 2, 5, 1)], -1)
    k1 = torch.cat([k, torch.full((1, 2, 7, 1), 4.0)], -1)
    torch.testing.assert_close(OA.attention_core(q1, k1, v, 0.3), base, rtol=1e-5, atol=1e-6)


def test_all_keys_masked_row_is_nan_and_zeroed_by_row_mask():
    p = _params(16)
    x = torch.randn(2, 4, 16)
    mask = torch.ones(2, 4, dtype=torch.bool)
    mask[1] = False
    out = OA.self_attention(x, p, 4, mask)
    assert torch.all(out[1] == 0)
    assert torch.isfinite(out[0]).all()


# -------------------------------------------------------------------- LayerNorm, block half
@pytest.mark.parametrize("affine", [False, True])
def test_layer_norm_matches_bruteforce_and_torch(affine):
    g = torch.Generator().manual_seed(21)
    x = torch.randn(5, 3, 48, generator=g) * 2.5 + 0.7
    w = torch.randn(48, generator=g) if affine else None
    b = torch.randn(48, generator=g) if affine else None
    got = OA.layer_norm(x, w, b, 1e-5)
    want = OA.layer_norm_bruteforce(x.numpy(), None if w is None else w.numpy(),
                                    None if b is None else b.numpy(), 1e-5)
    np.testing.assert_allclose(got.numpy(), want, rtol=2e-6, atol=2e-6)
    lib = torch.nn.functional.layer_norm(x, (48,), w, b, 1e-5)
    np.testing.assert_allclose(lib.numpy(), want, rtol=2e-6, atol=2e-6)


def test_layer_norm_closed_forms():
    w = torch.tensor([2.0, -3.0, 0.5, 1.0])
    b = torch.tensor([0.25, -1.0, 4.0, 0.0])
    const = torch.full((2, 4), 7.5)
    # a constant row has x - mean = 0 exactly: the output is the bias
    assert torch.equal(OA.layer_norm(const, w, b), b.expand(2, 4))
    # [a, -a] with eps = 0 has mean 0, biased variance a^2: normalised to [1, -1]
    two = torch.tensor([[3.0, -3.0], [-0.5, 0.5]])
    assert torch.allclose(OA.layer_norm(two, None, None, 0.0), torch.tensor([[1.0, -1.0], [-1.0, 1.0]]))
    # eps = 0: invariant under x -> c * x + s for c > 0, sign-flipped for c < 0
    x = torch.randn(3, 32, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    y = OA.layer_norm(x, None, None, 0.0)
    assert torch.allclose(OA.layer_norm(4.0 * x - 9.0, None, None, 0.0), y, atol=1e-12)
    assert torch.allclose(OA.layer_norm(-0.25 * x + 3.0, None, None, 0.0), -y, atol=1e-12)
    # eps inside the square root: [e, -e] rows shrink to e / sqrt(e^2 + eps)
    tiny = torch.tensor([[1e-3, -1e-3]], dtype=torch.float64)
    assert torch.allclose(OA.layer_norm(tiny, None, None, 1e-5),
                          torch.tensor([[1.0, -1.0]], dtype=torch.float64) * 1e-3 / (1e-6 + 1e-5) ** 0.5)


@pytest.mark.parametrize("mistake", ["unbiased", "eps_outside", "no_centering"])
def test_planted_layer_norm_mistakes_fail_the_pin(mistake):
    x = torch.randn(4, 16, generator=torch.Generator().manual_seed(8)) + 1.0
    want = OA.layer_norm_bruteforce(x.numpy(), None, None, 1e-2)
    mean = x.mean(-1, keepdim=True)
    var = x.var(-1, keepdim=True, unbiased=(mistake == "unbiased"))
    if mistake == "eps_outside":
        bad = (x - mean) / (torch.sqrt(var) + 1e-2)
    elif mistake == "no_centering":
        bad = x / torch.sqrt(var + 1e-2)
    else:
        bad = (x - mean) / torch.sqrt(var + 1e-2)
    assert not np.allclose(bad.numpy(), want, atol=1e-4)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("masked", [False, True])
def test_attention_half_matches_bruteforce(causal, masked):
    B, S, d, H = 2, 7, 16, 2
    g = torch.Generator().manual_seed(31)
    x = torch.randn(B, S, d, generator=g) * 1.5 + 0.3
    w, b = torch.randn(d, generator=g), torch.randn(d, generator=g)
    p = _params(d, seed=32)
    valid = torch.rand(B, S, generator=g) > 0.3 if masked else None
    if valid is not None:
        valid[:, 0] = True
    got = OA.attention_half(x, w, b, p, H, valid, causal)
    h = OA.layer_norm_bruteforce(x.numpy(), w.numpy(), b.numpy(), 1e-5)
    att = OA.self_attention_bruteforce(h, {k: v.numpy() for k, v in p.items()}, H, causal,
                                       None if valid is None else valid.numpy())
    np.testing.assert_allclose(got.numpy(), x.numpy() + att, rtol=2e-5, atol=2e-5)
    if valid is not None:
        # rows masked out of the attention output keep the residual input exactly
        assert torch.equal(got[~valid], x[~valid])


def test_attention_half_rounding_points():
    """round_to rounds the norm output, the attention output and the sum: with bf16 the
    result is representable in bf16 and differs from the fp32 half by rounding only."""
    g = torch.Generator().manual_seed(33)
    x = (torch.randn(1, 9, 16, generator=g)).to(torch.bfloat16)
    w, b = torch.randn(16, generator=g), torch.randn(16, generator=g)
    p = _params(16, seed=34)
    r = OA.attention_half(x, w, b, p, 2, round_to=torch.bfloat16)
    assert torch.equal(r, r.to(torch.bfloat16).float())
    f = OA.attention_half(x, w, b, p, 2)
    assert (r - f).abs().max() < 0.1 and not torch.equal(r, f)


def test_qkv_projection_equals_separate_projections():
    p = _params(16)
    x = torch.randn(2, 3, 16)
    qkv = OA.qkv_projection(x, p)
    for i, n in enumerate(("q_proj", "k_proj", "v_proj")):
        sep = torch.nn.functional.linear(x, p[f"{n}.weight"], p[f"{n}.bias"])
        torch.testing.assert_close(qkv[..., 16 * i:16 * (i + 1)], sep)


# ----------------------------------------------------------------------------- streamed
@pytest.mark.parametrize("causal", [False, True])
def test_streamed_equals_dense(causal):
    q, k, v = _qkv(2, 2, 37, 16, seed=7)
    dense = OA.attention_core(q, k, v, 0.25, causal)
    for qc, kc in ((2048, 8192), (5, 3), (1, 1)):
        got = OS.streamed_attention_core(q, k, v, 0.25, causal, q_chunk=qc, k_chunk=kc)
        torch.testing.assert_close(got, dense, rtol=1e-5, atol=1e-6)


def test_streamed_sampled_rows_use_absolute_positions():
    q, k, v = _qkv(1, 2, 40, 8, seed=9)
    dense = OA.attention_core(q, k, v, 0.3, causal=True)
    idx = torch.tensor([0, 3, 17, 39])
    got = OS.streamed_attention_core(q[:, :, idx], k, v, 0.3, True, q_chunk=3, k_chunk=7, q_index=idx)
    torch.testing.assert_close(got, dense[:, :, idx], rtol=1e-5, atol=1e-6)


# --------------------------------------------------------------------------------- int8
def test_quant_rows_hand_cases():
    t = np.array([[0.0, 0.0, 0.0, 0.0],          # zero row -> clamp: scale 1e-6/127
                  [1.0, -2.0, 0.5, 2.0],          # row max -> +-127
                  [127.0, 0.5, 1.5, -2.5]], np.float32)  # scale 1: .5 ties -> even
    q, s = OI.quant_rows(t)
    assert s[0] == np.float32(np.float32(1e-6) / np.float32(127.0))
    assert list(q[0]) == [0, 0, 0, 0]
    assert q[1, 1] == -127 and q[1, 3] == 127
    assert s[2] == np.float32(1.0)
    assert list(q[2]) == [127, 0, 2, -2]


def test_quant_weight_clamp_order():
    w = np.array([[0.0, 0.0], [254.0, -127.0]], np.float32)
    q, s = OI.quant_weight(w)
    assert s[0] == np.float32(1e-8)            # clamp applied after the /127
    assert s[1] == np.float32(2.0)
    assert list(q[1]) == [127, -64]            # -63.5 ties to even -> -64
    # the activation recipe clamps before dividing: different scale for a zero row
    _, sa = OI.quant_rows(w)
    assert sa[0] != s[0]


def test_int8_gemm_bruteforce():
    rng = np.random.default_rng(0)
    a = rng.integers(-128, 128, size=(5, 48), dtype=np.int8)
    w = rng.integers(-128, 128, size=(7, 48), dtype=np.int8)
    acc = OI.int8_gemm(a, w)
    want = np.zeros((5, 7), np.int64)
    for i in range(5):
        for j in range(7):
            want[i, j] = sum(int(a[i, kk]) * int(w[j, kk]) for kk in range(48))
    assert acc.dtype == np.int32
    np.testing.assert_array_equal(acc, want)
    # extreme values stay exact
    big = np.full((1, 4096), -128, np.int8)
    assert OI.int8_gemm(big, big)[0, 0] == 4096 * 128 * 128


def test_dequant_rounds_each_operation():
    acc = np.array([[16777217]], np.int32)      # not representable in fp32 -> rounds to even
    y = OI.dequant(acc, np.array([0.1], np.float32), np.array([3.0], np.float32),
                   np.array([0.25], np.float32))
    sc = np.float32(np.float32(0.1) * np.float32(3.0))
    want = np.float32(np.float32(np.float32(16777216.0) * sc) + np.float32(0.25))
    assert y[0, 0] == want


def test_quant_nonfinite_rows():
    """torch's amax/clamp propagate NaN into the row scale (k008_int8_gemm.py:150), and NaN
    quotients convert to code 0; an inf element makes the scale inf and every quotient 0 or NaN."""
    t = np.array([[1.0, np.nan, -3.0, 2.0], [1.0, -np.inf, 0.5, 2.0]], np.float32)
    q, s = OI.quant_rows(t)
    assert np.isnan(s[0]) and np.isinf(s[1])
    assert np.all(q == 0)
    qw, sw = OI.quant_weight(t)
    assert np.isnan(sw[0]) and np.isinf(sw[1]) and np.all(qw == 0)


def test_probability_rounding_point_with_one_hot_values():
    """attention_core(probs_dtype=...) rounds the normalised probabilities before P.V
    (torch_transformer_benchmark.py:111; k008_int8_gemm.py:108, :218): with one-hot value rows
    the context IS the probability row, so it must equal softmax rounded to fp16 exactly, and
    must not without the rounding (a dropped rounding point fails here)."""
    g = torch.Generator().manual_seed(3)
    S, hd = 24, 24
    q = torch.randn(1, 1, S, hd, generator=g)
    k = torch.randn(1, 1, S, hd, generator=g)
    v = torch.eye(S, hd)[None, None]
    scale = hd ** -0.5
    probs = torch.softmax(q @ k.transpose(-1, -2) * scale, dim=-1)
    got = OA.attention_core(q, k, v, scale, probs_dtype=torch.float16)
    assert torch.equal(got, probs.to(torch.float16).float())
    plain = OA.attention_core(q, k, v, scale)
    assert not torch.equal(plain, probs.to(torch.float16).float())
    # the int8 recipe's attention stage uses that rounding point: its context is fp16-rounded
    # P.V of fp16-rounded probabilities (checked through the same one-hot construction)
    import inspect
    assert "probs_dtype=torch.float16" in inspect.getsource(OI.int8_self_attention)


# ---------------------------------------------------------------------------- predicate
def test_predicate_clauses():
    ref = torch.tensor([1.0, 0.0, 100.0, 1.0, float("nan")])
    ok = OP.compare_outputs(ref[:4], torch.tensor([1.0019, 0.0019, 101.9, 1.0]))
    assert ok.passed
    bad_abs = OP.compare_outputs(torch.tensor([0.0]), torch.tensor([0.0021]))
    assert not bad_abs.passed
    bad_rel = OP.compare_outputs(torch.tensor([100.0]), torch.tensor([102.1]))
    assert not bad_rel.passed
    nan = OP.compare_outputs(ref, torch.tensor([1.0, 0.0, 100.0, 1.0, float("nan")]))
    assert not nan.passed and nan.failed_elements == 1
    inf = OP.compare_outputs(torch.tensor([1.0]), torch.tensor([float("inf")]))
    assert not inf.passed
    with pytest.raises(AssertionError):
        OP.compare_outputs(torch.zeros(2), torch.zeros(3))
