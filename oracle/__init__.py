"""CPU oracle for the attention-block hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the checker (or the timed CPU baseline). The product path
(``tiktok_techjam_2026_track3_amd``) never imports it and has no CPU fallback.

Contents (each function cites the reference file:line it restates):
  attention.py  dense fp32 torch-CPU restatement of ``BaselineSelfAttention.forward``, of the
                block's LayerNorm and of its attention half ``x + attention(norm1(x))``, and
                fp64 numpy brute forces used to pin them;
  streamed.py   chunk-wise online-softmax restatement of ``streamed_attention``;
  int8.py       numpy restatement of the W8A8 recipe (``_quant_rows``, ``_int8_pack``,
                ``_int8_linear``) with exact integer GEMM;
  predicate.py  the elementwise ``abs <= atol OR abs <= rtol*|ref|`` comparator;
  block.py      torch-CPU restatement of the rest of the block and model: exact GELU, the FFN
                half ``x + ffn_out(gelu(ffn_in(norm2(x))))`` with its row mask, the whole block
                and the L-layer model with the final norm, and fp64 brute forces;
  model.py      module-level restatement of the benchmark's transformer classes, used as the
                ``otb`` argument of the plugin contract in tests.

How each function is pinned (the reference ships no golden vectors for this path):
  attention.self_attention     fp64 brute force (per-row loops) + closed-form special cases
  attention.attention_core     same, plus softmax shift/permutation invariances
  attention.layer_norm         fp64 brute force, torch.nn.functional.layer_norm, closed forms
                               (constant row -> bias, two-element row -> -+1, shift/scale
                               invariance), planted-mistake checks
  attention.attention_half     fp64 brute force of norm + attention + residual
  streamed.*                   equals the dense restatement (fp32 reassociation only)
  int8.quant_rows / pack       hand-computed cases: zero row, row max -> +-127, .5 ties to even
  int8.int8_gemm               brute-force int64 loops on small shapes
  int8.int8_linear             hand-computed dequantisation on a 1x1x1 case
  int8.int8_transformer_block  within 0.5% RMS of block.transformer_block (int8 noise measured
                               0.35-0.39%); planted mistakes (GELU or the LayerNorms left out,
                               truncating quantisation) land outside; masked rows exact
  predicate.compare_outputs    hand-built cases for each clause (atol, rtol, NaN, inf)
  block.gelu                   math.erf fp64 brute force; x * Phi(x) at textbook Phi(1), Phi(2);
                               gelu(x) - gelu(-x) = x; the tanh approximation and a missing
                               1/sqrt(2) are caught
  block.ffn_half               fp64 brute force (per-row LayerNorm, np.dot, math.erf); planted
                               mistakes (no residual, mask before the residual, no norm) fail
  block.transformer_block /    equal the module classes of model.py (nn.LayerNorm, nn.Linear,
  block.transformer            F.gelu) and the composition attention_half -> ffn_half
Pins live in tests/test_oracle.py and tests/test_oracle_block.py.
"""
