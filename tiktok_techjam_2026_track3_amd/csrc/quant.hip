// Per-row symmetric int8 quantisation (activations per token, weights per output channel).
// One wave per row: pass 1 reduces |x| with 16-byte loads, pass 2 writes q = round_half_even(x / s)
// from the row held in registers (rows of 64 * 2^i 16-byte chunks, up to 16 per lane) or from a
// second read of the row (L1/L2 hit; other lengths). Division is IEEE fp32
// (hipcc's default correctly rounded divide), rounding is v_rndne_f32, so the output is
// bit-identical to the torch recipe it restates.
#include "common.h"

namespace {

template <typename T>
MI355_DEVINL void unpack16(const u32x4& v, float* out8);

template <>
MI355_DEVINL void unpack16<_Float16>(const u32x4& v, float* o) {
  const f16x8 h = __builtin_bit_cast(f16x8, v);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = static_cast<float>(h[e]);
}
template <>
MI355_DEVINL void unpack16<__bf16>(const u32x4& v, float* o) {
  const bf16x8 h = __builtin_bit_cast(bf16x8, v);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = static_cast<float>(h[e]);
}
template <>
MI355_DEVINL void unpack16<float>(const u32x4& v, float* o) {
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = __uint_as_float(v[e]);
}

// NaN-propagating maximum (IEEE maximum, as torch's amax and clamp): a row holding a NaN gets a
// NaN scale, as in the recipe (fmaxf would drop the NaN and give the row a finite scale).
MI355_DEVINL float nmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

MI355_DEVINL float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = nmax(v, __shfl_xor(v, off, 64));
  return v;
}

// round-half-even quotient -> int8; the quotients of a finite row lie in [-127, 127] (the scale is
// the row's amax / 127); a NaN quotient (NaN element or NaN scale) gives code 0, the value the
// recipe's float -> int8 conversion produces on the GPU
MI355_DEVINL uint32_t pack4_i8(const float* x, float s) {
  uint32_t w = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float r = __builtin_rintf(x[e] / s);
    r = r != r ? 0.f : fminf(fmaxf(r, -128.f), 127.f);
    w |= (static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xffu) << (8 * e);
  }
  return w;
}

template <typename T>
__global__ __launch_bounds__(256) void quant_rows_kernel(const T* __restrict__ X, int64_t ldx,
                                                         int8_t* __restrict__ Xq,
                                                         float* __restrict__ scale, int64_t M,
                                                         int64_t K, int mode) {
  constexpr int EPC = 16 / sizeof(T);  // elements per 16-byte load
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const T* xr = X + row * ldx;
  float amax = 0.f;
  // UNR loads in flight per lane (a loop of one load per trip waited for each load in turn)
  constexpr int UNR = 4;
  int64_t k = static_cast<int64_t>(lane) * EPC;
  for (; k + (UNR - 1) * 64 * EPC < K; k += UNR * 64 * EPC) {
    u32x4 v[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) v[u] = *reinterpret_cast<const u32x4*>(xr + k + u * 64 * EPC);
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      float f[8];
      unpack16<T>(v[u], f);
#pragma unroll
      for (int e = 0; e < EPC; ++e) amax = nmax(amax, fabsf(f[e]));
    }
  }
  for (; k < K; k += 64 * EPC) {
    float f[8];
    unpack16<T>(*reinterpret_cast<const u32x4*>(xr + k), f);
#pragma unroll
    for (int e = 0; e < EPC; ++e) amax = nmax(amax, fabsf(f[e]));
  }
  amax = wave_max(amax);
  // mode 0: clamp(amax, 1e-6) / 127 ; mode 1: clamp(amax / 127, 1e-8)
  const float s = mode == 0 ? nmax(amax, 1e-6f) / 127.0f : nmax(amax / 127.0f, 1e-8f);
  if (lane == 0) scale[row] = s;
  int8_t* qr = Xq + row * K;
  // 16 outputs per lane per step (one 16-byte store), two steps' loads in flight
  auto step = [&](int64_t kk) MI355_LAMBDA_INLINE {
    float f[16];
#pragma unroll
    for (int c = 0; c < 16 / EPC; ++c)
      unpack16<T>(*reinterpret_cast<const u32x4*>(xr + kk + c * EPC), f + c * EPC);
    u32x4 w;
#pragma unroll
    for (int d = 0; d < 4; ++d) w[d] = pack4_i8(f + 4 * d, s);
    *reinterpret_cast<u32x4*>(qr + kk) = w;
  };
  int64_t kq = static_cast<int64_t>(lane) * 16;
  for (; kq + 64 * 16 < K; kq += 2 * 64 * 16) {
    step(kq);
    step(kq + 64 * 16);
  }
  for (; kq < K; kq += 64 * 16) step(kq);
}

// The same with the row held in registers between the two passes (no second read): CPL
// 16-byte chunks per lane, K = CPL * 64 * (16 / sizeof(T)) exactly; each lane quantises its own
// chunks (8-byte stores of 8 codes for 16-bit inputs, 4-byte stores of 4 for fp32).
template <typename T, int CPL>
__global__ __launch_bounds__(256) void quant_rows_regs_kernel(const T* __restrict__ X, int64_t ldx,
                                                              int8_t* __restrict__ Xq,
                                                              float* __restrict__ scale, int64_t M,
                                                              int mode) {
  constexpr int EPC = 16 / sizeof(T);
  constexpr int64_t K = static_cast<int64_t>(CPL) * 64 * EPC;
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const T* xr = X + row * ldx + lane * EPC;
  u32x4 v[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) v[c] = *reinterpret_cast<const u32x4*>(xr + c * 64 * EPC);
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    float f[8];
    unpack16<T>(v[c], f);
#pragma unroll
    for (int e = 0; e < EPC; ++e) amax = nmax(amax, fabsf(f[e]));
  }
  amax = wave_max(amax);
  const float s = mode == 0 ? nmax(amax, 1e-6f) / 127.0f : nmax(amax / 127.0f, 1e-8f);
  if (lane == 0) scale[row] = s;
  int8_t* qr = Xq + row * K + lane * EPC;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    float f[8];
    unpack16<T>(v[c], f);
    if constexpr (EPC == 8) {
      u32x2 w = {pack4_i8(f, s), pack4_i8(f + 4, s)};
      *reinterpret_cast<u32x2*>(qr + c * 64 * EPC) = w;
    } else {
      *reinterpret_cast<uint32_t*>(qr + c * 64 * EPC) = pack4_i8(f, s);
    }
  }
}

template <typename T>
int launch_quant(const T* X, int64_t ldx, int8_t* Xq, float* scale, int64_t M, int64_t K, int mode,
                 hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((M + 3) / 4)), block(256);
  constexpr int64_t EPC = 16 / sizeof(T);
  // rows of up to 16 chunks per lane stay in registers (K = 8192 16-bit values: ~160 VGPRs, 3
  // waves per SIMD; 65536 x 4096 fp16: 235 -> 186 us). At 32 chunks (256 VGPRs, one wave per
  // SIMD) the two-pass kernel is faster (65536 x 16384: 765 against 1665 us).
  switch (K % (64 * EPC) == 0 ? K / (64 * EPC) : 0) {
    case 1: hipLaunchKernelGGL((quant_rows_regs_kernel<T, 1>), grid, block, 0, s, X, ldx, Xq, scale, M, mode); break;
    case 2: hipLaunchKernelGGL((quant_rows_regs_kernel<T, 2>), grid, block, 0, s, X, ldx, Xq, scale, M, mode); break;
    case 4: hipLaunchKernelGGL((quant_rows_regs_kernel<T, 4>), grid, block, 0, s, X, ldx, Xq, scale, M, mode); break;
    case 8: hipLaunchKernelGGL((quant_rows_regs_kernel<T, 8>), grid, block, 0, s, X, ldx, Xq, scale, M, mode); break;
    case 16: hipLaunchKernelGGL((quant_rows_regs_kernel<T, 16>), grid, block, 0, s, X, ldx, Xq, scale, M, mode); break;
    default: hipLaunchKernelGGL(quant_rows_kernel<T>, grid, block, 0, s, X, ldx, Xq, scale, M, K, mode); break;
  }
  return static_cast<int>(hipGetLastError());
}

}  // namespace

extern "C" int mi355_quant_rows_i8(int in_dtype, const void* X, int64_t ldx, int8_t* Xq,
                                   float* scale, int64_t M, int64_t K, int mode, void* stream) {
  if (M < 0 || K <= 0) return MI355_E_BAD_SIZE;
  if (M == 0) return MI355_OK;
  if (!X || !Xq || !scale) return MI355_E_NULL_POINTER;
  if (mode != 0 && mode != 1) return MI355_E_UNSUPPORTED;
  if (in_dtype != MI355_F32 && in_dtype != MI355_F16 && in_dtype != MI355_BF16)
    return MI355_E_BAD_DTYPE;
  const int64_t epc = in_dtype == MI355_F32 ? 4 : 8;
  if (K % 16 || ldx % epc || !aligned16(X) || !aligned16(Xq)) return MI355_E_ALIGNMENT;
  if (ldx < K) return MI355_E_BAD_SIZE;
  if ((M + 3) / 4 > 0x7fffffffLL) return MI355_E_BAD_SIZE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (in_dtype) {
    case MI355_F16:
      return launch_quant(static_cast<const _Float16*>(X), ldx, Xq, scale, M, K, mode, s);
    case MI355_BF16:
      return launch_quant(static_cast<const __bf16*>(X), ldx, Xq, scale, M, K, mode, s);
    default:
      return launch_quant(static_cast<const float*>(X), ldx, Xq, scale, M, K, mode, s);
  }
}
