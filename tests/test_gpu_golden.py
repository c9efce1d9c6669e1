"""The HIP path against the committed golden fixtures (tests/golden/*.npz).

Tolerance: the benchmark predicate ``abs <= 2e-3 OR abs <= 2e-2*|ref|`` (oracle.predicate) for
floating-point outputs; quantised activations, scales, int32 accumulators and the fp16 QKV of
the int8 path bit for bit; its end-to-end output within the requantisation bound of
tests/int8_requant.py.
"""
import numpy as np
import pytest
import torch

from golden_data import BLOCK_CASES, TORCH_DTYPE, load, params
from oracle import int8 as OI
from oracle.predicate import compare_outputs

import int8_requant
from test_gpu_block import INT8_E2E_PASS_FLOOR_FULL

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("name", BLOCK_CASES)
def test_block_against_fixture(gpu, name, causal):
    from tiktok_techjam_2026_track3_amd import SelfAttention
    c = load(name)
    dt = TORCH_DTYPE[str(c["dtype"])]
    x = torch.from_numpy(c["x"]).to(dt)
    B, S, d = x.shape
    mod = SelfAttention(d, int(c["heads"]))
    mod.load_state_dict(params(c, dt))
    mod = mod.to(gpu)
    mask = torch.from_numpy(c["mask"]).to(gpu)
    print(f"golden {name} causal={causal}", flush=True)
    with torch.inference_mode():
        out = mod(x.to(gpu), mask, causal)
    want = torch.from_numpy(c["out_causal" if causal else "out_noncausal"])
    r = compare_outputs(want, out)
    print(r.summary(), flush=True)
    assert r.passed, r.summary()
    assert torch.all(out.cpu()[~torch.from_numpy(c["mask"])] == 0)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_hd128_against_fixture(gpu, causal):
    from tiktok_techjam_2026_track3_amd import ops
    c = load("attn_f16_hd128_b1s80h2")
    q, k, v = (torch.from_numpy(c[n]).to(gpu) for n in "qkv")
    mask = torch.from_numpy(c["mask"]).to(gpu)
    with torch.inference_mode():
        o = ops.attention(q, k, v, scale=128 ** -0.5, causal=causal, key_valid=mask)
    r = compare_outputs(torch.from_numpy(c["ctx_causal" if causal else "ctx_noncausal"]), o)
    print(r.summary(), flush=True)
    assert r.passed, r.summary()


def test_int8_block_against_fixture(gpu):
    from tiktok_techjam_2026_track3_amd import Int8SelfAttention, ops
    c = load("int8_block_b1s64_d128h2")
    x = torch.from_numpy(c["x"])
    B, S, d = x.shape
    T = B * S
    mod = Int8SelfAttention(d, int(c["heads"]))
    mod.load_state_dict(params(c))
    mod = mod.to(gpu)
    keep = {}
    with torch.inference_mode():
        out = mod.run(x.to(gpu), None, False, keep=keep)
        # raw int32 accumulators of the QKV GEMM through the C-ABI
        w_i8, s_w = mod._int8_weights(gpu)[:2]
        acc = torch.empty(T, 3 * d, dtype=torch.int32, device=gpu)
        ops.linear_i8(keep["x_i8"], w_i8, keep["x_scale"], s_w, acc_out=acc, want_out=False)
    np.testing.assert_array_equal(keep["x_i8"].cpu().numpy(), c["x_i8"])
    np.testing.assert_array_equal(keep["x_scale"].cpu().numpy(), c["x_scale"])
    np.testing.assert_array_equal(acc.cpu().numpy(), c["qkv_acc"])
    np.testing.assert_array_equal(keep["qkv"].cpu().numpy(), c["qkv16"])
    r = compare_outputs(torch.from_numpy(c["ctx16"]).float(), keep["ctx"].reshape(T, d))
    print("ctx:", r.summary(), flush=True)
    assert r.passed, r.summary()
    pk = OI.pack_block(params(c))
    frac, stats = int8_requant.check(keep["ctx"].reshape(T, d), torch.from_numpy(c["ctx16"]),
                                     pk["out_w"], pk["out_s"], pk["out_b"], out.reshape(T, d))
    print("end to end vs the quantised recipe:", stats, flush=True)
    assert frac >= INT8_E2E_PASS_FLOOR_FULL, stats


@pytest.mark.parametrize("mode,q,s", [(0, "q_act", "s_act"), (1, "q_w", "s_w")])
def test_quant_rows_against_fixture(gpu, mode, q, s):
    from tiktok_techjam_2026_track3_amd import ops
    c = load("quant_rows_cases")
    xq, sx = ops.quant_rows_i8(torch.from_numpy(c["x"]).to(gpu), mode=mode)
    np.testing.assert_array_equal(xq.cpu().numpy(), c[q])
    np.testing.assert_array_equal(sx.cpu().numpy(), c[s])
