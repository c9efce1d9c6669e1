"""The oracle still reproduces the committed golden fixtures (tests/golden/make_golden.py).

Float outputs are compared at 1e-5 relative (torch-CPU fp32 GEMMs may reassociate across
machines and thread counts); integer outputs and scales must match exactly.
"""
import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import int8 as OI
from golden_data import BLOCK_CASES, TORCH_DTYPE, load, params


@pytest.mark.parametrize("name", BLOCK_CASES)
def test_block_fixtures(name):
    c = load(name)
    dt = TORCH_DTYPE[str(c["dtype"])]
    p = params(c)
    # stored values are exactly representable in the case's dtype
    for v in list(p.values()) + [torch.from_numpy(c["x"])]:
        assert torch.equal(v.float(), v.to(dt).float())
    x = torch.from_numpy(c["x"]).float()
    mask = torch.from_numpy(c["mask"])
    for causal in (False, True):
        ref = OA.self_attention(x, p, int(c["heads"]), mask, causal=causal).numpy()
        want = c["out_causal" if causal else "out_noncausal"]
        np.testing.assert_allclose(ref, want, rtol=1e-5, atol=1e-6)
        assert np.all(want[~c["mask"]] == 0)


def test_attention_fixture():
    c = load("attn_f16_hd128_b1s80h2")
    q, k, v = (torch.from_numpy(c[n]).float().transpose(1, 2) for n in "qkv")
    for causal in (False, True):
        o = OA.attention_core(q, k, v, 128 ** -0.5, causal, torch.from_numpy(c["mask"]))
        np.testing.assert_allclose(o.transpose(1, 2).numpy(),
                                   c["ctx_causal" if causal else "ctx_noncausal"], rtol=1e-5, atol=1e-6)


def test_int8_fixture():
    c = load("int8_block_b1s64_d128h2")
    p = params(c)
    x = c["x"]
    T, d = x.shape[0] * x.shape[1], x.shape[2]
    xq, sx = OI.quant_rows(x.astype(np.float32).reshape(T, d))
    np.testing.assert_array_equal(xq, c["x_i8"])
    np.testing.assert_array_equal(sx, c["x_scale"])
    pk = OI.pack_block(p)
    np.testing.assert_array_equal(OI.int8_gemm(xq, pk["qkv_w"]), c["qkv_acc"])
    want = OI.int8_self_attention(torch.from_numpy(x), p, int(c["heads"]), False)
    np.testing.assert_array_equal(want["qkv16"].numpy(), c["qkv16"])
    np.testing.assert_allclose(want["ctx16"].float().numpy(), c["ctx16"].astype(np.float32),
                               rtol=1e-3, atol=1e-4)


def test_quant_fixture():
    c = load("quant_rows_cases")
    q0, s0 = OI.quant_rows(c["x"])
    q1, s1 = OI.quant_weight(c["x"])
    for a, b in ((q0, "q_act"), (s0, "s_act"), (q1, "q_w"), (s1, "s_w")):
        np.testing.assert_array_equal(a, c[b])
    # the hand-made tie row: scale 1.0, so x.5 rounds to even
    assert c["s_act"][4] == np.float32(1.0)
    assert list(c["q_act"][4][:6]) == [127, 0, 2, 2, 0, -2]
