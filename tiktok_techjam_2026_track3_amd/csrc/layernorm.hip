// Row LayerNorm (nn.LayerNorm over the last dimension) for gfx950:
//   y = (x - mean) * rstd * gamma + beta,  rstd = 1 / sqrt(var + eps),  var biased (divide by K)
// Statistics and the affine map are fp32; y is rounded once to the input dtype. G lanes per row
// (G = 64: one wave per row; rows of at most 32 16-byte vectors share a wave, 64 / G rows per
// wave, so that short rows keep every lane busy), the row held in registers as 16-byte vectors
// (up to G * NV vectors), two-pass mean / variance. HBM-bound: reads the row once and writes it
// once.
#include "common.h"

namespace {

// sum over the G lanes of a row group (lanes g*G .. g*G + G - 1): butterfly over offsets < G.
// A row of n < G vectors leaves lanes n.. at 0, so the sum has the bits of the 64-lane tree.
template <int G>
MI355_DEVINL float group_sum(float v) {
#pragma unroll
  for (int off = G / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// TO: output type (the input type, or fp16 for an fp32 input: the fp16 operands of an fp32
// model's projections)
template <typename T, int NV, int G, typename TO = T>
__global__ __launch_bounds__(256) void layernorm_rows(const T* __restrict__ X, int64_t ldx,
                                                      const T* __restrict__ gamma,
                                                      const T* __restrict__ beta, float eps,
                                                      TO* __restrict__ Y, int64_t ldy, int64_t M,
                                                      int K, const uint8_t* __restrict__ row_valid) {
  constexpr int EPV = 16 / static_cast<int>(sizeof(T));  // elements per 16-byte vector
  typedef T tv __attribute__((ext_vector_type(EPV)));
  typedef TO tov __attribute__((ext_vector_type(EPV)));
  const int lane = threadIdx.x % G;  // lane within the row group
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (256 / G) + threadIdx.x / G;
  if (row >= M) return;  // the row group leaves together (its shuffles stay inside it)
  const int nvec = K / EPV;
  if (row_valid != nullptr && row_valid[row] == 0) {
    // masked row: zeros (the masked_fill that follows the final norm)
    TO* yr = Y + row * ldy;
    for (int vi = lane; vi < nvec; vi += G) *reinterpret_cast<tov*>(yr + static_cast<int64_t>(vi) * EPV) = tov{};
    return;
  }
  const T* xr = X + row * ldx;

  float xs[NV][EPV];
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int vi = lane + G * j;
    tv v = {};
    if (vi < nvec) v = *reinterpret_cast<const tv*>(xr + static_cast<int64_t>(vi) * EPV);
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      xs[j][e] = to_f32(v[e]);
      sum += xs[j][e];
    }
  }
  const float mean = group_sum<G>(sum) / static_cast<float>(K);
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    if (lane + G * j < nvec) {
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        const float d = xs[j][e] - mean;
        sq += d * d;
      }
    }
  }
  const float var = group_sum<G>(sq) / static_cast<float>(K);
  const float rstd = 1.0f / sqrtf(var + eps);

  TO* yr = Y + row * ldy;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int vi = lane + G * j;
    if (vi >= nvec) continue;
    tv gv, bv;
    if (gamma) gv = *reinterpret_cast<const tv*>(gamma + static_cast<int64_t>(vi) * EPV);
    if (beta) bv = *reinterpret_cast<const tv*>(beta + static_cast<int64_t>(vi) * EPV);
    tov out;
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      float y = (xs[j][e] - mean) * rstd;
      if (gamma) y = y * to_f32(gv[e]);
      if (beta) y = y + to_f32(bv[e]);
      out[e] = from_f32<TO>(y);
    }
    *reinterpret_cast<tov*>(yr + static_cast<int64_t>(vi) * EPV) = out;
  }
}

// Row statistics only: stats[2 row] = mean, stats[2 row + 1] = rstd, computed exactly as in
// layernorm_rows (the same loads, sums and rounding), for GEMMs that fold the normalisation into
// their epilogue (mi355_layernorm_gemm_bias). Reads the row once, writes 8 bytes. A row whose
// variance is exactly 0 (every element equals the mean, so its normalised values are exactly
// beta) gets rstd 0: the folded epilogue then yields the bias term alone instead of
// 1/sqrt(eps) times the fp32 rounding residue of x W'^T - mean colsum.
template <typename T, int NV, int G>
__global__ __launch_bounds__(256) void layernorm_stats(const T* __restrict__ X, int64_t ldx, float eps,
                                                       float* __restrict__ stats, int64_t M, int K) {
  constexpr int EPV = 16 / static_cast<int>(sizeof(T));
  typedef T tv __attribute__((ext_vector_type(EPV)));
  const int lane = threadIdx.x % G;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (256 / G) + threadIdx.x / G;
  if (row >= M) return;
  const int nvec = K / EPV;
  const T* xr = X + row * ldx;
  float xs[NV][EPV];
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int vi = lane + G * j;
    tv v = {};
    if (vi < nvec) v = *reinterpret_cast<const tv*>(xr + static_cast<int64_t>(vi) * EPV);
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      xs[j][e] = to_f32(v[e]);
      sum += xs[j][e];
    }
  }
  const float mean = group_sum<G>(sum) / static_cast<float>(K);
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    if (lane + G * j < nvec) {
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        const float d = xs[j][e] - mean;
        sq += d * d;
      }
    }
  }
  const float var = group_sum<G>(sq) / static_cast<float>(K);
  if (lane == 0) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<f32x2*>(stats + 2 * row) = f32x2{mean, var > 0.f ? 1.0f / sqrtf(var + eps) : 0.f};
  }
}

// lanes per row: rows of at most 8 / 16 / 32 vectors take that many lanes (8 / 4 / 2 rows per
// wave), longer rows a whole wave
inline int lanes_per_row(int64_t nvec) { return nvec <= 8 ? 8 : nvec <= 16 ? 16 : nvec <= 32 ? 32 : 64; }

template <typename T>
int launch_stats(const void* X, int64_t ldx, float eps, float* stats, int64_t M, int64_t K,
                 hipStream_t s) {
  constexpr int EPV = 16 / static_cast<int>(sizeof(T));
  const int64_t nvec = K / EPV;
  const int g = lanes_per_row(nvec);
  const int64_t blocks = (M + 256 / g - 1) / (256 / g);
  if (blocks > 0x7fffffffLL) return MI355_E_BAD_SIZE;
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  const T* x = static_cast<const T*>(X);
  const int k = static_cast<int>(K);
  if (g == 8)
    hipLaunchKernelGGL((layernorm_stats<T, 1, 8>), grid, block, 0, s, x, ldx, eps, stats, M, k);
  else if (g == 16)
    hipLaunchKernelGGL((layernorm_stats<T, 1, 16>), grid, block, 0, s, x, ldx, eps, stats, M, k);
  else if (g == 32)
    hipLaunchKernelGGL((layernorm_stats<T, 1, 32>), grid, block, 0, s, x, ldx, eps, stats, M, k);
  else if (nvec <= 64)
    hipLaunchKernelGGL((layernorm_stats<T, 1, 64>), grid, block, 0, s, x, ldx, eps, stats, M, k);
  else if (nvec <= 128)
    hipLaunchKernelGGL((layernorm_stats<T, 2, 64>), grid, block, 0, s, x, ldx, eps, stats, M, k);
  else if (nvec <= 256)
    hipLaunchKernelGGL((layernorm_stats<T, 4, 64>), grid, block, 0, s, x, ldx, eps, stats, M, k);
  else if (nvec <= 512)
    hipLaunchKernelGGL((layernorm_stats<T, 8, 64>), grid, block, 0, s, x, ldx, eps, stats, M, k);
  else
    hipLaunchKernelGGL((layernorm_stats<T, 16, 64>), grid, block, 0, s, x, ldx, eps, stats, M, k);
  return static_cast<int>(hipGetLastError());
}

template <typename T, typename TO = T>
int launch_ln(const void* X, int64_t ldx, const void* gamma, const void* beta, float eps, void* Y,
              int64_t ldy, int64_t M, int64_t K, const uint8_t* rv, hipStream_t s) {
  constexpr int EPV = 16 / static_cast<int>(sizeof(T));
  const int64_t nvec = K / EPV;
  const int gl = lanes_per_row(nvec);
  const int64_t blocks = (M + 256 / gl - 1) / (256 / gl);
  if (blocks > 0x7fffffffLL) return MI355_E_BAD_SIZE;
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  const T* x = static_cast<const T*>(X);
  const T* g = static_cast<const T*>(gamma);
  const T* b = static_cast<const T*>(beta);
  TO* y = static_cast<TO*>(Y);
  const int k = static_cast<int>(K);
  if (gl == 8)
    hipLaunchKernelGGL((layernorm_rows<T, 1, 8, TO>), grid, block, 0, s, x, ldx, g, b, eps, y, ldy, M, k, rv);
  else if (gl == 16)
    hipLaunchKernelGGL((layernorm_rows<T, 1, 16, TO>), grid, block, 0, s, x, ldx, g, b, eps, y, ldy, M, k, rv);
  else if (gl == 32)
    hipLaunchKernelGGL((layernorm_rows<T, 1, 32, TO>), grid, block, 0, s, x, ldx, g, b, eps, y, ldy, M, k, rv);
  else if (nvec <= 64)
    hipLaunchKernelGGL((layernorm_rows<T, 1, 64, TO>), grid, block, 0, s, x, ldx, g, b, eps, y, ldy, M, k, rv);
  else if (nvec <= 128)
    hipLaunchKernelGGL((layernorm_rows<T, 2, 64, TO>), grid, block, 0, s, x, ldx, g, b, eps, y, ldy, M, k, rv);
  else if (nvec <= 256)
    hipLaunchKernelGGL((layernorm_rows<T, 4, 64, TO>), grid, block, 0, s, x, ldx, g, b, eps, y, ldy, M, k, rv);
  else if (nvec <= 512)
    hipLaunchKernelGGL((layernorm_rows<T, 8, 64, TO>), grid, block, 0, s, x, ldx, g, b, eps, y, ldy, M, k, rv);
  else
    hipLaunchKernelGGL((layernorm_rows<T, 16, 64, TO>), grid, block, 0, s, x, ldx, g, b, eps, y, ldy, M, k, rv);
  return static_cast<int>(hipGetLastError());
}

}  // namespace

// Library-internal (declared in common.h): the statistics pass of mi355_layernorm_gemm_bias.
// Arguments are validated by the caller.
int mi355_internal_ln_stats(int dtype, const void* X, int64_t ldx, float eps, float* stats,
                            int64_t M, int64_t K, hipStream_t s) {
  switch (dtype) {
    case MI355_F16: return launch_stats<_Float16>(X, ldx, eps, stats, M, K, s);
    case MI355_BF16: return launch_stats<__bf16>(X, ldx, eps, stats, M, K, s);
    default: return launch_stats<float>(X, ldx, eps, stats, M, K, s);
  }
}

extern "C" int mi355_layernorm_masked(int dtype, const void* X, int64_t ldx, const void* gamma,
                                      const void* beta, float eps, void* Y, int64_t ldy, int64_t M,
                                      int64_t K, const uint8_t* row_valid, void* stream) {
  if (M < 0 || K <= 0) return MI355_E_BAD_SIZE;
  if (M == 0) return MI355_OK;
  if (!X || !Y) return MI355_E_NULL_POINTER;
  if (dtype != MI355_F32 && dtype != MI355_F16 && dtype != MI355_BF16) return MI355_E_BAD_DTYPE;
  if (!(eps >= 0.f)) return MI355_E_BAD_SIZE;
  const int64_t epv = dtype == MI355_F32 ? 4 : 8;
  if (K % epv || ldx % epv || ldy % epv || !aligned16(X) || !aligned16(Y) ||
      (gamma && !aligned16(gamma)) || (beta && !aligned16(beta)))
    return MI355_E_ALIGNMENT;
  if (ldx < K || ldy < K) return MI355_E_BAD_SIZE;
  if (K / epv > 64 * 16) return MI355_E_UNSUPPORTED;  // row must fit the registers of one wave
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MI355_F16: return launch_ln<_Float16>(X, ldx, gamma, beta, eps, Y, ldy, M, K, row_valid, s);
    case MI355_BF16: return launch_ln<__bf16>(X, ldx, gamma, beta, eps, Y, ldy, M, K, row_valid, s);
    default: return launch_ln<float>(X, ldx, gamma, beta, eps, Y, ldy, M, K, row_valid, s);
  }
}

extern "C" int mi355_layernorm(int dtype, const void* X, int64_t ldx, const void* gamma,
                               const void* beta, float eps, void* Y, int64_t ldy, int64_t M,
                               int64_t K, void* stream) {
  return mi355_layernorm_masked(dtype, X, ldx, gamma, beta, eps, Y, ldy, M, K, nullptr, stream);
}

extern "C" int mi355_layernorm_cvt(int dtype, int out_dtype, const void* X, int64_t ldx,
                                   const void* gamma, const void* beta, float eps, void* Y,
                                   int64_t ldy, int64_t M, int64_t K, void* stream) {
  if (out_dtype == dtype)
    return mi355_layernorm_masked(dtype, X, ldx, gamma, beta, eps, Y, ldy, M, K, nullptr, stream);
  if (dtype != MI355_F32 || out_dtype != MI355_F16) {
    if ((dtype != MI355_F32 && dtype != MI355_F16 && dtype != MI355_BF16) ||
        (out_dtype != MI355_F32 && out_dtype != MI355_F16 && out_dtype != MI355_BF16))
      return MI355_E_BAD_DTYPE;
    return MI355_E_UNSUPPORTED;
  }
  if (M < 0 || K <= 0) return MI355_E_BAD_SIZE;
  if (M == 0) return MI355_OK;
  if (!X || !Y) return MI355_E_NULL_POINTER;
  if (!(eps >= 0.f)) return MI355_E_BAD_SIZE;
  // fp32 rows read as 16-byte vectors of 4, fp16 rows written as 8-byte vectors of 4
  if (K % 4 || ldx % 4 || ldy % 4 || !aligned16(X) || (reinterpret_cast<uintptr_t>(Y) & 7u) ||
      (gamma && !aligned16(gamma)) || (beta && !aligned16(beta)))
    return MI355_E_ALIGNMENT;
  if (ldx < K || ldy < K) return MI355_E_BAD_SIZE;
  if (K / 4 > 64 * 16) return MI355_E_UNSUPPORTED;  // row must fit the registers of one wave
  return launch_ln<float, _Float16>(X, ldx, gamma, beta, eps, Y, ldy, M, K, nullptr,
                                    static_cast<hipStream_t>(stream));
}
