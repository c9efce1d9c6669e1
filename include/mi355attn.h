/*
 * mi355attn.h — C-ABI of libmi355attn.so, the gfx950 (MI355X) attention-block hot path.
 *
 * The reference implements this path as Python/PyTorch ops plus Triton kernels; its only native
 * binding is the inline CUDA extension `nq_launch(int cfg, Tensor X, W, Bias, LnW, LnB, Out,
 * int64 tokens, int64 D)` launched on the current stream
 * (Project/kernels/k024_cuda_tuned.py:201-245). Every entry point below replaces one stage of
 * `BaselineSelfAttention.forward` (torch_transformer_benchmark.py:85-122) or of its optimised
 * restatements, and is cited at its declaration.
 *
 * Conventions (all entry points):
 *   - plain device pointers, element strides and sizes; no framework types;
 *   - `stream` is a hipStream_t passed as void* (NULL = the legacy default stream); kernels are
 *     enqueued asynchronously, nothing is allocated, nothing synchronises the host, so a caller
 *     may capture the calls in a hipGraph;
 *   - return 0 on success, a negative MI355_E* code on an argument error (nothing launched),
 *     or a positive hipError_t from the launch.
 */
#ifndef MI355ATTN_H
#define MI355ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types */
#define MI355_F32 0
#define MI355_F16 1
#define MI355_BF16 2

/* argument-error status codes (negative) */
#define MI355_OK 0
#define MI355_E_NULL_POINTER (-1)   /* a required pointer is NULL */
#define MI355_E_BAD_SIZE (-2)       /* a size is negative or exceeds the supported range */
#define MI355_E_BAD_DTYPE (-3)      /* dtype code not supported by this entry point */
#define MI355_E_ALIGNMENT (-4)      /* pointer or leading dimension violates 16-byte vector access */
#define MI355_E_HEAD_DIM (-5)       /* head_dim not in {8, 16, 32, 48, 64, 80, 96, 128, 192, 256} */
#define MI355_E_UNSUPPORTED (-6)    /* argument combination not supported */

/* Library version, e.g. 100 for 0.1.0. */
int mi355_version(void);

/* Static description of a status code (never NULL). */
const char* mi355_status_string(int status);

/*
 * Dense projection  C[M,N] = A[M,K] · W[N,K]^T + bias[N]   (nn.Linear semantics).
 * Replaces q_proj/k_proj/v_proj/out_proj (torch_transformer_benchmark.py:93-95, :118) and the
 * packed-QKV F.linear of the optimised route (Project/submission/dispatcher_region.py:789-792,
 * :1025, :1085). A and W share in_dtype (F32, F16, BF16); C has out_dtype: any of the three for
 * 16-bit inputs, F32 or F16 for F32 inputs (F16 carries an fp32 model's q/k/v into the fp16
 * attention core; F32 out of a 16-bit product returns its context projection to fp32). bias
 * is fp32 or NULL.
 * Accumulation and the bias add are fp32; C is rounded once (round-to-nearest-even).
 * Rows m with row_valid[m] == 0 are written as exact zeros (the output-row mask of
 * torch_transformer_benchmark.py:120-121); row_valid may be NULL (all rows valid).
 * Requirements: K % (16 / sizeof(elem)) == 0, lda/ldw multiples of that, 16-byte aligned A, W.
 */
int mi355_gemm_bias(int in_dtype, int out_dtype, const void* A, int64_t lda, const void* W,
                    int64_t ldw, const float* bias, void* C, int64_t ldc, int64_t M, int64_t N,
                    int64_t K, const uint8_t* row_valid, void* stream);

/*
 * Streamed scaled-dot-product attention forward with online softmax; never forms S_q x S_k.
 * Replaces scores/causal mask/key mask/softmax/P·V/head merge of BaselineSelfAttention.forward
 * (torch_transformer_benchmark.py:97-117), the Triton kernels `_sub_attn_fwd` and
 * `_sub_attn_heads` (Project/submission/dispatcher_region.py:217-291, :418-556) and the streamed
 * oracle `streamed_attention` (Project/tools/shape14_eval.py:201-236).
 *
 * Q, K, V, O are 4-D [B, S, H, head_dim] views given by element strides (batch, seq, head);
 * the head_dim stride must be 1. The packed [B, S, 3*d] QKV output of mi355_gemm_bias is read
 * in place with seq stride 3*d. O is written in the caller's layout ([B, S, H, hd] makes the
 * head merge free). Scores use `scale` (head_dim^-0.5 in the reference); softmax is fp32;
 * probabilities are rounded to the input dtype before P·V (torch_transformer_benchmark.py:111).
 * causal != 0 masks key j > query i (triu(diagonal=1), :99-103).
 * key_valid (nullable) is a [B, S_k] byte mask with batch stride key_valid_sb; keys with 0 are
 * excluded (:105-108). A query row whose keys are all excluded produces NaN, as softmax over an
 * all -inf row does in the reference.
 * Supported: dtype F32, F16, BF16 with head_dim 8, 16, 32, 48, 64, 80, 96, 128, 192 or 256
 * (the benchmark's official shapes use 8, 32, 64, 128 and 256: Project/shapes.json). F16/BF16
 * with head_dim 64 or 128 run on the matrix cores; the other 16-bit head dims and every F32
 * problem run on a vector-ALU kernel with fp32 arithmetic (16-bit probabilities are rounded the
 * same way).
 */
int mi355_attn_fwd(int dtype, const void* Q, const void* K, const void* V, void* O, int64_t B,
                   int64_t H, int64_t S_q, int64_t S_k, int64_t head_dim,
                   const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                   const int64_t* o_strides, float scale, int causal, const uint8_t* key_valid,
                   int64_t key_valid_sb, void* stream);

/*
 * mi355_attn_fwd with a caller-provided workspace (same interface and results contract; replaces
 * the same reference code). On the matrix-core kernel (F16 / BF16, head_dim 32, 64, 128) a
 * workspace of at least B * H * ceil(S_k / 256) * 4 bytes (4-byte aligned) holds the key-norm
 * bounds max |k| per 256-key chunk of every head (a chunk is one 256-query work-group tile),
 * computed by a pass over K on the same stream before the attention launch. A wave whose every
 * query satisfies |c q| max|k| - mu <= 8 (c = scale * log2 e, mu its lazily moved running
 * maximum) can never move mu again, so it skips the per-tile row maxima for the rest of its
 * sweep: the output is bit-identical to mi355_attn_fwd. Causal work-groups reduce only the
 * chunks of the keys they visit (up to the end of their query tile), so no output row depends
 * on a key or query past the end of its 256-row tile. On work-groups whose keys are all valid: a
 * wave whose bound keeps every score within +-T (log2 units; T = 11 non-causal, 8 causal) from
 * the start runs with mu = 0 and no row maxima at all (the max-free sweep; causal calls over the
 * keys before the work-group's first query, in query tiles whose key range reaches 32768 keys);
 * its output then differs from mi355_attn_fwd only in rounding, under the same error bound. When the workspace also holds the redo flags (from the next 256-byte boundary
 * after the bounds, one int per 256-query work-group: mi355_attn_workspace_bytes), a wave whose
 * bounds exceed T may instead fix mu at bound - T in advance (the offset sweep); a work-group in
 * which a row's probability sum then stays below 1 is recomputed on the exact path by a second
 * launch on the same stream. Same error bound. With a key mask and room for the redo flags, the
 * bound pass also marks the chunks holding an invalid key; work-groups that visit one leave the
 * first launch at once and are run by the second launch with the key mask applied (decided on
 * the device: an all-true mask costs the same as no mask, and nothing waits for the host).
 * workspace may be NULL (then the same as mi355_attn_fwd); a smaller non-NULL workspace than
 * the bounds need is MI355_E_BAD_SIZE. Causal calls with a key mask use it only with room for
 * the redo flags. The workspace is scratch: its contents on return are unspecified, and calls
 * that share one workspace must be stream-ordered.
 */
int mi355_attn_fwd_ws(int dtype, const void* Q, const void* K, const void* V, void* O, int64_t B,
                      int64_t H, int64_t S_q, int64_t S_k, int64_t head_dim,
                      const int64_t* q_strides, const int64_t* k_strides,
                      const int64_t* v_strides, const int64_t* o_strides, float scale,
                      int causal, const uint8_t* key_valid, int64_t key_valid_sb,
                      void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Workspace bytes the library recommends for mi355_attn_fwd_ws on this problem: the key-norm
 * bounds rounded up to 256 bytes plus B * H * ceil(S_q / 256) redo flags of 4 bytes, when the
 * problem runs on the matrix-core kernel with S_k >= 32768 (shorter key ranges do not repay
 * the extra pass over K), else 0 (call without a workspace).
 */
int64_t mi355_attn_workspace_bytes(int dtype, int64_t B, int64_t H, int64_t S_q, int64_t S_k,
                                   int64_t head_dim);

/*
 * The same workspace size at any key length (bounds and redo flags), for callers that want the
 * bound pass and the sweeps below the recommended length; 0 when the problem does not run on
 * the matrix-core kernel. Replaces the same reference code as mi355_attn_fwd.
 */
int64_t mi355_attn_workspace_bytes_forced(int dtype, int64_t B, int64_t H, int64_t S_q,
                                          int64_t S_k, int64_t head_dim);

/*
 * mi355_attn_fwd_ws with two more controls, for a caller whose QKV projection already wrote the
 * key-norm bounds (mi355_gemm_bias_kbound / mi355_layernorm_gemm_bias_kbound, same format and
 * the same bits as the bound pass; replaces the same reference code as mi355_attn_fwd):
 *   bounds_ready != 0: the workspace's bound section already holds the bounds of this K (and,
 *     with a key mask, its chunk marks), so no bound pass is launched; the workspace must
 *     then be given and hold at least the bounds;
 *   causal_sweep_min_keys: causal work-groups take the max-free / offset sweeps only when their
 *     key range [0, end of their 256-row query tile) holds at least this many keys (>= 0;
 *     mi355_attn_fwd_ws uses 32768). Whatever the value, whether a row is swept depends on its
 *     own query tile only, so a prefix run still gives the full run's rows bit for bit when
 *     both runs use the same value and both have the workspace.
 */
int mi355_attn_fwd_kb(int dtype, const void* Q, const void* K, const void* V, void* O, int64_t B,
                      int64_t H, int64_t S_q, int64_t S_k, int64_t head_dim,
                      const int64_t* q_strides, const int64_t* k_strides,
                      const int64_t* v_strides, const int64_t* o_strides, float scale,
                      int causal, const uint8_t* key_valid, int64_t key_valid_sb,
                      void* workspace, int64_t workspace_bytes, int bounds_ready,
                      int64_t causal_sweep_min_keys, void* stream);

/*
 * Per-row symmetric int8 quantisation of X[M,K] (row stride ldx) into Xq[M,K] (contiguous) and
 * scale[M] (fp32). mode 0 = activation recipe `_quant_rows`
 * (Project/kernels/k008_int8_gemm.py:148-151): s = max(amax, 1e-6) / 127.
 * mode 1 = weight recipe `_int8_pack` (k008_int8_gemm.py:154-158): s = max(amax / 127, 1e-8).
 * Both then store q = round_half_even(x / s) with IEEE fp32 division; X dtype is F32/F16/BF16
 * (converted exactly to fp32 first). K % (16 / sizeof(elem)) == 0 and ldx likewise.
 */
int mi355_quant_rows_i8(int in_dtype, const void* X, int64_t ldx, int8_t* Xq, float* scale,
                        int64_t M, int64_t K, int mode, void* stream);

/*
 * W8A8 projection: acc[M,N] = A_i8[M,K] · W_i8[N,K]^T in exact int32, then
 * C = out_dtype( fp32(acc) * (s_a[m] * s_w[n]) + bias[n] ) with separately rounded fp32
 * multiply/multiply/add, matching `_int8_linear` (Project/kernels/k008_int8_gemm.py:181-185;
 * torch._int_mm + dequant). W is stored [N, K] (K contiguous) — the transpose of the
 * reference's `[K, N]` cache (k008_int8_gemm.py:158) — so both MFMA operands are K-major.
 * out_dtype is F32, F16 or BF16; bias (fp32) may be NULL; C may be NULL when acc_out is given.
 * acc_out (nullable, [M,N] int32, row stride N) receives the raw accumulators before
 * dequantisation. row_valid as for mi355_gemm_bias. K % 16 == 0, A and W contiguous rows.
 */
int mi355_gemm_i8(const int8_t* A, const int8_t* W, const float* s_a, const float* s_w,
                  const float* bias, int out_dtype, void* C, int64_t ldc, int32_t* acc_out,
                  int64_t M, int64_t N, int64_t K, const uint8_t* row_valid, void* stream);

/* epilogue flags of mi355_gemm_i8_epilogue */
#define MI355_EPI_GELU 1         /* C = gelu(projection), exact (erf) form */
#define MI355_EPI_ZERO_MASKED 2  /* with R: rows with row_valid[m] == 0 are written as zeros */

/*
 * mi355_gemm_i8 with the epilogues of the int8 transformer block (block_forward,
 * Project/kernels/k008_int8_gemm.py:189-234), so that block runs whole on the kernels:
 *   epi = MI355_EPI_GELU, R = NULL:  C = gelu(y)        `F.gelu(_int8_linear(h2, f1))` (:228-229)
 *   epi = 0, R given:                C = R + y, rows with row_valid[m] == 0 keep R
 *                                    (`attn_out.masked_fill(...); x = x + attn_out`, :221-225)
 *   epi = MI355_EPI_ZERO_MASKED, R:  C = R + y, rows with row_valid[m] == 0 are zero
 *                                    (`x = x + out; x.masked_fill(...)`, :230-233)
 * where y = out_dtype(fp32(acc) * (s_a[m] * s_w[n]) + bias[n]) as in mi355_gemm_i8 (masked rows
 * of y are 0), and GELU / the residual sum are evaluated in fp32 from y and rounded once to
 * out_dtype. R (nullable) is [M, N] of out_dtype with row stride ldr and may alias C. GELU
 * with R is rejected (MI355_E_UNSUPPORTED). Otherwise as mi355_gemm_i8 (no acc_out).
 */
int mi355_gemm_i8_epilogue(const int8_t* A, const int8_t* W, const float* s_a, const float* s_w,
                           const float* bias, int out_dtype, void* C, int64_t ldc, const void* R,
                           int64_t ldr, int64_t M, int64_t N, int64_t K,
                           const uint8_t* row_valid, int epi, void* stream);

/*
 * Row LayerNorm: Y[m,:] = (X[m,:] - mean) * rstd * gamma + beta over the last dimension (K), with
 * fp32 mean, biased variance and rstd = 1 / sqrt(var + eps), Y rounded once to dtype. Replaces
 * `self.norm1(x)` of BaselineTransformerBlock.forward (torch_transformer_benchmark.py:139;
 * nn.LayerNorm(d_model), :128), the input of the attention block. dtype F32/F16/BF16 for X, Y,
 * gamma and beta (gamma/beta nullable: 1 / 0, as elementwise_affine=False). K % (16 / sizeof(elem))
 * == 0, K <= 8192 (16-bit) / 4096 (fp32), 16-byte aligned pointers; Y may equal X (in place).
 */
int mi355_layernorm(int dtype, const void* X, int64_t ldx, const void* gamma, const void* beta,
                    float eps, void* Y, int64_t ldy, int64_t M, int64_t K, void* stream);

/*
 * nn.LayerNorm as mi355_layernorm, with the normalised rows written in another type:
 * out_dtype == dtype is mi355_layernorm; dtype F32 with out_dtype F16 computes in fp32 and rounds
 * the result once to fp16 (the fp16 operand of an fp32 model's projection: the reference's fast
 * route runs fp32 models on fp16 tiles, Project/submission/dispatcher_region.py:1017-1091, with
 * the LayerNorm fused into its QKV kernel, :343-399). Other pairs: MI355_E_UNSUPPORTED.
 * F32 -> F16: K, ldx, ldy multiples of 4, X 16-byte and Y 8-byte aligned.
 */
int mi355_layernorm_cvt(int dtype, int out_dtype, const void* X, int64_t ldx, const void* gamma,
                        const void* beta, float eps, void* Y, int64_t ldy, int64_t M, int64_t K,
                        void* stream);

/*
 * Projection with the block's residual add fused into its epilogue:
 *   C = R + out_dtype(A · W^T + bias)
 * i.e. `x + self.attention(...)` of BaselineTransformerBlock.forward
 * (torch_transformer_benchmark.py:139) with the attention's out_proj (:118) and its output-row
 * mask (:120-121): the projection is rounded to out_dtype first and the sum rounded again (the
 * reference adds two tensors of that dtype); rows with row_valid[m] == 0 give C = R (the masked
 * attention row is zero). R has out_dtype and row stride ldr; R may be C (in place). Otherwise as
 * mi355_gemm_bias.
 */
int mi355_gemm_bias_residual(int in_dtype, int out_dtype, const void* A, int64_t lda, const void* W,
                             int64_t ldw, const float* bias, const void* R, int64_t ldr, void* C,
                             int64_t ldc, int64_t M, int64_t N, int64_t K, const uint8_t* row_valid,
                             void* stream);

/*
 * FFN input projection with the exact GELU fused into its epilogue:
 *   C = out_dtype( gelu( out_dtype(A · W^T + bias) ) ),  gelu(x) = x * 0.5 * (1 + erf(x / sqrt 2))
 * i.e. `F.gelu(self.ffn_in(h), approximate="none")` of BaselineTransformerBlock.forward
 * (torch_transformer_benchmark.py:141; ffn_in = nn.Linear(d_model, ffn_dim), :131): the linear
 * output is rounded to out_dtype (the nn.Linear output tensor), GELU is evaluated in fp32 on it and
 * rounded again. Arguments as mi355_gemm_bias without the row mask.
 */
int mi355_gemm_bias_gelu(int in_dtype, int out_dtype, const void* A, int64_t lda, const void* W,
                         int64_t ldw, const float* bias, void* C, int64_t ldc, int64_t M, int64_t N,
                         int64_t K, void* stream);

/*
 * FFN output projection with the residual add and the block's trailing row mask fused:
 *   C = R + out_dtype(A · W^T + bias) for rows with row_valid[m] != 0, C = 0 for the others
 * i.e. `x = x + self.ffn_out(...)` followed by `x.masked_fill(~valid_token_mask[..., None], 0)`
 * (torch_transformer_benchmark.py:141-144; ffn_out = nn.Linear(ffn_dim, d_model), :132).
 * row_valid may be NULL (no row is masked). Otherwise as mi355_gemm_bias_residual.
 */
int mi355_gemm_bias_residual_zero_masked(int in_dtype, int out_dtype, const void* A, int64_t lda,
                                         const void* W, int64_t ldw, const float* bias,
                                         const void* R, int64_t ldr, void* C, int64_t ldc,
                                         int64_t M, int64_t N, int64_t K,
                                         const uint8_t* row_valid, void* stream);

/*
 * mi355_layernorm with a row mask: rows with row_valid[m] == 0 are written as zeros. Replaces
 * `self.norm2(x)` (torch_transformer_benchmark.py:141, row_valid NULL) and the model's
 * `self.final_norm(x)` followed by `x.masked_fill(~valid_token_mask[..., None], 0)` (:168-171).
 * row_valid may be NULL. Otherwise as mi355_layernorm.
 */
int mi355_layernorm_masked(int dtype, const void* X, int64_t ldx, const void* gamma, const void* beta,
                           float eps, void* Y, int64_t ldy, int64_t M, int64_t K,
                           const uint8_t* row_valid, void* stream);

/*
 * LayerNorm folded into a projection:
 *   C = out_dtype( LayerNorm(X) · W^T + b )   with LayerNorm(X) = (X - mean) * rstd * gamma + beta
 * Replaces `self.norm1(x)` feeding the packed QKV projection (torch_transformer_benchmark.py:139,
 * :93-95) -- the reference's fused LN-prologue QKV kernels `nq_launch(cfg, X, W, Bias, LnW, LnB,
 * Out, tokens, D)` (Project/kernels/k024_cuda_tuned.py:201-234) and `_sub_norm_qkv`
 * (Project/submission/dispatcher_region.py:343-399) -- and, with epi = MI355_EPI_GELU,
 * `F.gelu(self.ffn_in(self.norm2(x)))` (:141). The normalised rows are never written: the caller
 * passes the folded weight Wf[n, k] = W[n, k] * gamma[k] (rounded to in_dtype, row stride ldw),
 * colsum[n] = sum_k Wf[n, k] (fp32) and bias[n] = b[n] + sum_k beta[k] W[n, k] (fp32, NULL = 0);
 * one pass computes each row's mean and rstd = 1 / sqrt(var + eps) (biased variance, fp32; 0 for a
 * row of equal elements, whose normalised values are exactly beta) into `stats` (caller workspace
 * of 2 * M floats, 8-byte aligned, overwritten), and the projection of the raw X forms
 * rstd * (X·Wf^T - mean * colsum) + bias in its epilogue (then the exact GELU of that value
 * rounded to out_dtype, with MI355_EPI_GELU). X·Wf^T accumulates in fp32, so a row whose mean is
 * large against its spread (|mean| * rstd >> 1) carries an extra error of about
 * rstd * |mean| * sum_k |Wf[n, k]| * K / 16 * 2^-24. out_dtype is in_dtype, or F16 for a BF16
 * input (the attention core type of a bf16 model). Requirements as mi355_gemm_bias, and
 * K / (16 / sizeof(elem)) <= 1024.
 */
int mi355_layernorm_gemm_bias(int in_dtype, int out_dtype, const void* X, int64_t ldx,
                              const void* W, int64_t ldw, const float* colsum, const float* bias,
                              float eps, float* stats, void* C, int64_t ldc, int64_t M, int64_t N,
                              int64_t K, int epi, void* stream);

/*
 * Key-norm bounds from the QKV projection's epilogue. mi355_gemm_bias (and
 * mi355_layernorm_gemm_bias, with epi = 0) of the packed QKV projection
 * (torch_transformer_benchmark.py:93-95; Project/submission/dispatcher_region.py:1025) that also
 * writes, for the K block -- output columns [k_col0, k_col0 + n_heads * head_dim) of the M =
 * B * seq_len token rows -- the key-norm bounds that mi355_attn_fwd_kb reads with bounds_ready:
 * key_bounds[(b * n_heads + h) * (seq_len / 256) + i] = max |k| over keys 256 i .. 256 i + 255
 * of head h of batch row b, computed from the rounded outputs in the order of the attention's
 * bound pass (the same bits), with the sign bit set when key_valid ([B, seq_len] bytes,
 * nullable) has a 0 among those keys. key_bounds is the bound section of the attention's
 * workspace (4-byte aligned). Requires 16-bit inputs and outputs, head_dim 32, 64 or 128,
 * seq_len, k_col0 and n_heads * head_dim multiples of 256, 16-byte aligned output rows, and a
 * problem that runs on the 256 x 256-tile kernel; otherwise MI355_E_UNSUPPORTED with nothing
 * launched (the projection part of the LayerNorm-folded form may have run its statistics
 * pass), and the caller runs the plain projection and lets the attention run its bound pass.
 */
int mi355_gemm_bias_kbound(int in_dtype, int out_dtype, const void* A, int64_t lda,
                           const void* W, int64_t ldw, const float* bias, void* C, int64_t ldc,
                           int64_t M, int64_t N, int64_t K, float* key_bounds, int64_t k_col0,
                           int64_t n_heads, int64_t head_dim, int64_t seq_len,
                           const uint8_t* key_valid, void* stream);
int mi355_layernorm_gemm_bias_kbound(int in_dtype, int out_dtype, const void* X, int64_t ldx,
                                     const void* W, int64_t ldw, const float* colsum,
                                     const float* bias, float eps, float* stats, void* C,
                                     int64_t ldc, int64_t M, int64_t N, int64_t K,
                                     float* key_bounds, int64_t k_col0, int64_t n_heads,
                                     int64_t head_dim, int64_t seq_len,
                                     const uint8_t* key_valid, void* stream);

/* largest M of mi355_layernorm_gemm_bias_noalloc (its statistics array: 8 MiB per GPU) */
#define MI355_NOALLOC_MAX_ROWS (1 << 20)

/*
 * mi355_layernorm_gemm_bias without the `stats` workspace: the row statistics go to a file-scope
 * device array of the library (MI355_NOALLOC_MAX_ROWS rows, 8 MiB per GPU, held until the process
 * ends), so the call allocates nothing and takes no workspace. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation). M > MI355_NOALLOC_MAX_ROWS returns
 * MI355_E_BAD_SIZE. All calls on one GPU share that array: calls that overlap on one GPU (on
 * different streams, or from several threads) race and must be ordered by the caller. The first
 * call on a device looks the array's address up (hipGetSymbolAddress) and keeps it. Otherwise as
 * mi355_layernorm_gemm_bias, with the same kernels and results.
 */
int mi355_layernorm_gemm_bias_noalloc(int in_dtype, int out_dtype, const void* X, int64_t ldx,
                                      const void* W, int64_t ldw, const float* colsum,
                                      const float* bias, float eps, void* C, int64_t ldc, int64_t M,
                                      int64_t N, int64_t K, int epi, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MI355ATTN_H */
