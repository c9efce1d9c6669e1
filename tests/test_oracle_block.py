"""Pins of the CPU oracle for the rest of the transformer block (oracle/block.py).

Each check is chosen so a plausible mistake fails it: the tanh approximation of GELU, a missing
1/sqrt(2), a dropped residual, the mask applied before the residual, an unnormalised FFN input.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import block as OB
from oracle import model as OM


def _ffn_params(d, f, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return {
        "norm2.weight": (1 + 0.1 * torch.randn(d, generator=g)).to(dtype),
        "norm2.bias": (0.1 * torch.randn(d, generator=g)).to(dtype),
        "ffn_in.weight": (torch.randn(f, d, generator=g) / math.sqrt(d)).to(dtype),
        "ffn_in.bias": (0.1 * torch.randn(f, generator=g)).to(dtype),
        "ffn_out.weight": (torch.randn(d, f, generator=g) / math.sqrt(f)).to(dtype),
        "ffn_out.bias": (0.1 * torch.randn(d, generator=g)).to(dtype),
    }


def test_gelu_matches_erf_bruteforce():
    x = torch.linspace(-12, 12, 4801, dtype=torch.float64)
    np.testing.assert_allclose(OB.gelu(x).numpy(), OB.gelu_bruteforce(x.numpy()), rtol=1e-13, atol=1e-15)
    x32 = torch.linspace(-8, 8, 2001, dtype=torch.float32)
    # fp32: 1 + erf(x / sqrt 2) cancels for x < -5 (as in torch's own fp32 GELU): absolute error
    # up to ~2e-7 there
    np.testing.assert_allclose(OB.gelu(x32).numpy(), OB.gelu_bruteforce(x32.numpy()), rtol=2e-6, atol=3e-7)


def test_gelu_closed_forms():
    x = torch.tensor([0.0, 1.0, -1.0, 2.0, 10.0, -10.0, 40.0, -40.0], dtype=torch.float64)
    y = OB.gelu(x).numpy()
    assert y[0] == 0.0
    # x * Phi(x) with the textbook normal CDF values Phi(1) = 0.8413447460685429,
    # Phi(2) = 0.9772498680518208
    assert abs(y[1] - 0.8413447460685429) < 1e-15
    assert abs(y[2] + (1 - 0.8413447460685429)) < 1e-15
    assert abs(y[3] - 2 * 0.9772498680518208) < 1e-14
    assert abs(y[4] - 10.0) < 1e-15 and abs(y[5]) < 1e-20
    assert y[6] == 40.0 and y[7] == 0.0
    # gelu(x) - gelu(-x) = x (since Phi(-x) = 1 - Phi(x))
    z = torch.linspace(-6, 6, 1201, dtype=torch.float64)
    np.testing.assert_allclose((OB.gelu(z) - OB.gelu(-z)).numpy(), z.numpy(), atol=1e-14)


def test_gelu_planted_tanh_approximation_is_caught():
    x = torch.linspace(-6, 6, 1201, dtype=torch.float64)
    tanh = 0.5 * x * (1 + torch.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))
    exact = OB.gelu_bruteforce(x.numpy())
    assert np.abs(tanh.numpy() - exact).max() > 1e-4  # the approximation differs visibly
    no_sqrt2 = x * 0.5 * (1 + torch.erf(x))
    assert np.abs(no_sqrt2.numpy() - exact).max() > 1e-2


@pytest.mark.parametrize("masked", [False, True])
def test_ffn_half_matches_bruteforce(masked):
    B, S, d, f = 2, 7, 16, 40
    p = _ffn_params(d, f, seed=3)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, S, d, generator=g, dtype=torch.float64)
    valid = None
    if masked:
        valid = torch.ones(B, S, dtype=torch.bool)
        valid[0, 5:] = False
        valid[1, 0] = False
    got = OB.ffn_half(x, p, valid).numpy()
    want = OB.ffn_half_bruteforce(x.numpy(), {k: v.numpy() for k, v in p.items()},
                                  None if valid is None else valid.numpy())
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    if masked:
        assert np.all(got[~valid.numpy()] == 0)


def test_ffn_half_planted_mistakes_are_caught():
    B, S, d, f = 1, 5, 8, 24
    p = _ffn_params(d, f, seed=5)
    x = torch.randn(B, S, d, generator=torch.Generator().manual_seed(6), dtype=torch.float64)
    valid = torch.tensor([[True, True, False, True, True]])
    want = OB.ffn_half_bruteforce(x.numpy(), {k: v.numpy() for k, v in p.items()}, valid.numpy())
    pn = {k: v.numpy() for k, v in p.items()}
    # dropped residual
    no_res = OB.ffn_half_bruteforce(np.zeros_like(x.numpy()), pn) + 0  # LN of zeros -> bias path
    assert np.abs(no_res - want).max() > 1e-3
    # mask applied to the input instead of the output: masked rows keep x + ffn(0-row)
    xm = x.masked_fill(~valid[..., None], 0)
    wrong = OB.ffn_half(xm, p).numpy()
    assert np.abs(wrong - want).max() > 1e-3
    # FFN on x instead of norm2(x)
    p_id = dict(p, **{"norm2.weight": torch.ones(d, dtype=torch.float64), "norm2.bias": torch.zeros(d, dtype=torch.float64)})
    h = torch.nn.functional.layer_norm(x, (d,))
    assert not torch.allclose(h, x)
    got = OB.ffn_half(x, p, valid).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    assert np.abs(OB.ffn_half(x, p_id, valid).numpy() - want).max() > 1e-3


def test_ffn_half_rounding_points():
    B, S, d, f = 1, 6, 16, 32
    p = _ffn_params(d, f, seed=7, dtype=torch.float32)
    x = torch.randn(B, S, d, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).float()
    r = OB.ffn_half(x, p, round_to=torch.bfloat16)
    assert torch.equal(r, r.to(torch.bfloat16).float())  # every output is bf16-representable
    f32 = OB.ffn_half(x, p)
    assert (r - f32).abs().max() < 0.1 and not torch.equal(r, f32)


@pytest.mark.parametrize("causal", [False, True])
def test_block_and_model_match_torch_modules(causal):
    """The composed restatement equals the module classes of oracle/model.py, which run
    nn.LayerNorm, nn.Linear and F.gelu (torch_transformer_benchmark.py:125-172). fp32: the
    attention restatement computes in fp32, as the reference's softmax does."""
    cfg = OM.TransformerConfig(batch_size=2, seq_len=9, d_model=16, num_heads=2, ffn_dim=24,
                               num_layers=2, causal=causal)
    torch.manual_seed(11)
    model = OM.BaselineTransformer(cfg)
    with torch.no_grad():
        for prm in model.parameters():
            prm.add_(0.05 * torch.randn_like(prm))
    x = torch.randn(2, 9, 16)
    valid = torch.ones(2, 9, dtype=torch.bool)
    valid[1, 6:] = False
    params = {k: v.detach() for k, v in model.state_dict().items()}
    with torch.no_grad():
        want_block = model.layers[0](x, valid, causal)
        want = model(x, valid)
    got_block = OB.transformer_block(x, {k[len("layers.0."):]: v for k, v in params.items()
                                         if k.startswith("layers.0.")}, 2, valid, causal)
    torch.testing.assert_close(got_block, want_block, rtol=1e-5, atol=1e-5)
    got = OB.transformer(x, params, 2, 2, valid, causal)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
    assert torch.all(got[~valid] == 0)
    # the block is the attention half followed by the FFN half
    blk = {k[len("layers.0."):]: v for k, v in params.items() if k.startswith("layers.0.")}
    x1 = OA.attention_half(x, blk["norm1.weight"], blk["norm1.bias"],
                           {k[len("attention."):]: v for k, v in blk.items() if k.startswith("attention.")},
                           2, valid, causal)
    torch.testing.assert_close(OB.ffn_half(x1, blk, valid), got_block, rtol=0, atol=0)


def _int8_block_case(causal, seed=21):
    from oracle import int8 as OI
    cfg = OM.TransformerConfig(batch_size=2, seq_len=12, d_model=32, num_heads=2, ffn_dim=64,
                               num_layers=1, causal=causal)
    torch.manual_seed(seed)
    model = OM.BaselineTransformer(cfg)
    with torch.no_grad():
        for prm in model.parameters():
            prm.add_(0.05 * torch.randn_like(prm))
    x = torch.randn(2, 12, 32)
    valid = torch.ones(2, 12, dtype=torch.bool)
    valid[1, 7:] = False
    blk = {k[len("layers.0."):]: v.detach() for k, v in model.state_dict().items()
           if k.startswith("layers.0.")}
    return OI, x, valid, blk


def _rel_rms(got, want, valid):
    e = (got - want)[valid]
    return float(e.pow(2).mean().sqrt() / want[valid].pow(2).mean().sqrt())


# int8 recipe vs float block, relative RMS over the valid rows: measured 0.35-0.39% (seeds 5, 21,
# 77, causal or not); activations truncated instead of rounded: 0.66-0.76%
INT8_REL_RMS = 0.005


@pytest.mark.parametrize("causal", [False, True])
def test_int8_block_close_to_float_block(causal):
    """oracle.int8.int8_transformer_block (k008_int8_gemm.py:189-234) against the float block
    restatement: per-token int8 activations and per-channel int8 weights add about 0.4% RMS noise
    to the block output. Masked rows of the attention half keep x exactly and masked output rows
    are exact zeros."""
    OI, x, valid, blk = _int8_block_case(causal)
    got = OI.int8_transformer_block(x, blk, 2, valid, causal)
    want = OB.transformer_block(x, blk, 2, valid, causal)
    rel = _rel_rms(got["out"], want, valid)
    print(f"int8 vs float block: relative RMS {rel:.4f}")
    assert rel <= INT8_REL_RMS
    assert float((got["out"] - want).abs().max()) <= 0.01 * float(want.abs().max())
    assert torch.all(got["out"][~valid] == 0)
    assert torch.equal(got["x1"].view(2, 12, 32)[~valid], x[~valid])
    h = OA.layer_norm(x.reshape(-1, 32), blk["norm1.weight"], blk["norm1.bias"])
    torch.testing.assert_close(got["h"], h, rtol=0, atol=0)
    assert got["qkv16"].dtype == torch.float16 and got["ctx16"].dtype == torch.float16


def test_int8_block_planted_mistakes_are_caught(monkeypatch):
    """The closeness check above separates the recipe from plausible mistakes planted in the
    oracle: GELU left out, both LayerNorms left out, and activations quantised by truncation
    instead of round-half-even."""
    OI, x, valid, blk = _int8_block_case(False)
    want = OB.transformer_block(x, blk, 2, valid, False)

    def rel():
        return _rel_rms(OI.int8_transformer_block(x, blk, 2, valid, False)["out"], want, valid)

    assert rel() <= INT8_REL_RMS
    with monkeypatch.context() as m:
        m.setattr(OB, "gelu", lambda t: t)
        assert rel() > INT8_REL_RMS
    with monkeypatch.context() as m:
        m.setattr(OA, "layer_norm", lambda t, w, b, eps=1e-5: t)
        assert rel() > INT8_REL_RMS
    with monkeypatch.context() as m:
        def quant_trunc(t):
            t = np.asarray(t, dtype=np.float32)
            s = (np.maximum(np.abs(t).max(axis=-1), np.float32(1e-6)) / np.float32(127.0)).astype(np.float32)
            return np.trunc(t / s[:, None]).astype(np.int8), s
        m.setattr(OI, "quant_rows", quant_trunc)
        assert rel() > INT8_REL_RMS
