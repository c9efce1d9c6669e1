"""The allocation-free entry point mi355_layernorm_gemm_bias_noalloc (row statistics in the
library's file-scope device array) against mi355_layernorm_gemm_bias (caller workspace), called
through the C-ABI: the same kernels, so bit-identical outputs, on two calls in a row -- the
second with a smaller input, so its rows overwrite only part of the array the first call
filled. (The size limit is rejected on the host before anything is launched:
tests/test_abi_cpu.py.)"""
import ctypes as C
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

F16, BF16, F32 = 1, 2, 0
CODE = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}


def _case(M, N, K, dtype, seed):
    from tiktok_techjam_2026_track3_amd import ops
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, K, generator=g) + 0.5 * torch.randn(M, 1, generator=g)).to(dtype).cuda()
    gamma = (1 + 0.3 * torch.randn(K, generator=g)).to(dtype).cuda()
    beta = (0.2 * torch.randn(K, generator=g)).to(dtype).cuda()
    w = (torch.randn(N, K, generator=g) / math.sqrt(K)).to(dtype).cuda()
    b = (0.1 * torch.randn(N, generator=g)).cuda()
    wf, colsum, bf = ops.fold_layernorm(w, b, gamma, beta, dtype)
    return x, wf, colsum, bf


def _call(fn_name, x, wf, colsum, bf, odt, gelu, stats=None):
    from tiktok_techjam_2026_track3_amd import _lib
    M, K = x.shape
    N = wf.shape[0]
    out = torch.full((M, N), float("nan"), device=x.device, dtype=odt)
    stream = torch.cuda.current_stream().cuda_stream
    fn = getattr(_lib.lib(), fn_name)
    args = [CODE[x.dtype], CODE[odt], x.data_ptr(), x.stride(0), wf.data_ptr(), wf.stride(0),
            colsum.data_ptr(), bf.data_ptr(), C.c_float(1e-5)]
    if stats is not None:
        args.append(stats.data_ptr())
    args += [out.data_ptr(), out.stride(0), M, N, K, 1 if gelu else 0, stream]
    rc = fn(*args)
    return rc, out


@pytest.mark.parametrize("dtype,odt", [(torch.float16, torch.float16), (torch.bfloat16, torch.float16),
                                       (torch.float32, torch.float32)])
@pytest.mark.parametrize("gelu", [False, True])
def test_noalloc_matches_workspace_entry_point(dtype, odt, gelu):
    for call, (M, N, K) in enumerate([(2048, 768, 256), (300, 768, 256)]):
        print(f"noalloc {dtype}->{odt} gelu={gelu} call {call}: M={M} N={N} K={K}", flush=True)
        x, wf, colsum, bf = _case(M, N, K, dtype, seed=100 * call + K)
        stats = torch.empty(M, 2, device="cuda")
        rc_ref, ref = _call("mi355_layernorm_gemm_bias", x, wf, colsum, bf, odt, gelu, stats)
        rc, out = _call("mi355_layernorm_gemm_bias_noalloc", x, wf, colsum, bf, odt, gelu)
        torch.cuda.synchronize()
        assert rc_ref == 0 and rc == 0, (rc_ref, rc)
        assert torch.isfinite(ref).all()
        assert torch.equal(out, ref)

