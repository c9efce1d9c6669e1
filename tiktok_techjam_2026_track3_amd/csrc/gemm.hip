// Projection GEMMs of the attention block on gfx950 MFMA:
//   C[M,N] = A[M,K] · W[N,K]^T + bias[N]                      (fp16 / bf16 / fp32, fp32 accumulate)
//   C[M,N] = fp32(A_i8 · W_i8^T) * (s_a[m] * s_w[n]) + bias[n] (int8 x int8 -> exact int32)
// Both operands are K-major (nn.Linear weight layout), so every MFMA fragment is one 16-byte LDS
// read per lane. Work-group tile BM x BN, waves arranged WM x WN, each wave owning
// (BM/WM) x (BN/WN) as 32x32 MFMA tiles. K is staged 128 bytes per row per step (64 fp16,
// 128 int8, 32 fp32 elements), double-buffered in LDS with an XOR swizzle on 16-byte chunks.
#include "common.h"

namespace {

struct GemmArgs {
  const void* A;
  const void* W;
  const float* bias;  // fp32, nullable
  void* C;
  int32_t* acc_out;  // int8 only (nullable)
  const float* s_a;  // int8 only
  const float* s_w;  // int8 only
  const uint8_t* row_valid;
  int64_t lda, ldw, ldc;
  int64_t M, N, K;
  int out_dtype;
};

template <typename TO>
MI355_DEVINL void store_out(void* C, int64_t idx, float v) {
  static_cast<TO*>(C)[idx] = from_f32<TO>(v);
}

constexpr int CH = 8;  // 16-byte chunks per LDS row per K step (128 bytes)

// Chunk swizzle: conflict-free 16-byte fragment reads for 8- or 16-lane LDS phases.
MI355_DEVINL int swz8(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// XCD-aware work-group order: the dispatcher deals work-groups round-robin to the 8 XCDs, so
// hand each XCD a contiguous range of logical tiles (shared A rows / W columns stay in its L2),
// then walk tiles in groups of GROUP_M tile-rows.
MI355_DEVINL void tile_coords(int64_t pid, int64_t ntm, int64_t ntn, int64_t& tm, int64_t& tn) {
  constexpr int GROUP_M = 8;
  const int64_t total = ntm * ntn;
  const int64_t q = total / 8, r = total % 8;
  const int64_t x = pid % 8, j = pid / 8;
  const int64_t logical = x * q + (x < r ? x : r) + j;
  const int64_t in_group = GROUP_M * ntn;
  const int64_t group = logical / in_group;
  const int64_t first_m = group * GROUP_M;
  const int64_t gsize = (ntm - first_m) < GROUP_M ? (ntm - first_m) : GROUP_M;
  const int64_t w = logical % in_group;
  tm = first_m + w % gsize;
  tn = w / gsize;
}

template <typename T, typename TO, int BM, int BN, int WM, int WN, bool INT8>
__global__ __launch_bounds__(WM* WN * 64) void gemm_kernel(GemmArgs p) {
  using MF = Mfma<T>;
  using frag = typename MF::frag;
  using acc_t = typename MF::acc;
  constexpr int NT = WM * WN * 64;
  constexpr int EPC = MF::ELEMS_PER_CHUNK;
  constexpr int BK = CH * EPC;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int A_LOADS = BM * CH / NT, B_LOADS = BN * CH / NT;
  static_assert((BM * CH) % NT == 0 && (BN * CH) % NT == 0, "loader shape");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile");

  __shared__ u32x4 lds[2][(BM + BN) * CH];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t ntm = (p.M + BM - 1) / BM, ntn = (p.N + BN - 1) / BN;
  int64_t tmi, tni;
  tile_coords(blockIdx.x, ntm, ntn, tmi, tni);
  const int64_t m0 = tmi * BM, n0 = tni * BN;

  const char* __restrict__ Ab = static_cast<const char*>(p.A);
  const char* __restrict__ Wb = static_cast<const char*>(p.W);
  constexpr int ES = sizeof(T);

  u32x4 ra[A_LOADS], rb[B_LOADS];
  auto load_global = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int idx = tid + i * NT, row = idx / CH, ch = idx % CH;
      const int64_t gm = m0 + row, gk = k0 + ch * EPC;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (gm < p.M && gk < p.K)
        v = *reinterpret_cast<const u32x4*>(Ab + (gm * p.lda + gk) * ES);
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int idx = tid + i * NT, row = idx / CH, ch = idx % CH;
      const int64_t gn = n0 + row, gk = k0 + ch * EPC;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (gn < p.N && gk < p.K)
        v = *reinterpret_cast<const u32x4*>(Wb + (gn * p.ldw + gk) * ES);
      rb[i] = v;
    }
  };
  auto store_lds = [&](int s) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int idx = tid + i * NT, row = idx / CH, ch = idx % CH;
      lds[s][row * CH + (ch ^ swz8(row))] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int idx = tid + i * NT, row = idx / CH, ch = idx % CH;
      lds[s][(BM + row) * CH + (ch ^ swz8(row))] = rb[i];
    }
  };

  acc_t acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0;

  const int nk = static_cast<int>((p.K + BK - 1) / BK);
  load_global(0);
  store_lds(0);
  __syncthreads();

  const int g = lane >> 5, l32 = lane & 31;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_global(static_cast<int64_t>(kt + 1) * BK);
#pragma unroll
    for (int j = 0; j < CH / 2; ++j) {
      const int c = 2 * j + g;
      frag fa[TM], fb[TN];
#pragma unroll
      for (int a = 0; a < TM; ++a) {
        const int row = wm * WTM + a * 32 + l32;
        u32x4 v = lds[cur][row * CH + (c ^ swz8(row))];
        fa[a] = __builtin_bit_cast(frag, v);
      }
#pragma unroll
      for (int b = 0; b < TN; ++b) {
        const int row = wn * WTN + b * 32 + l32;
        u32x4 v = lds[cur][(BM + row) * CH + (c ^ swz8(row))];
        fb[b] = __builtin_bit_cast(frag, v);
      }
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = MF::mma(fa[a], fb[b], acc[a][b]);
    }
    if (kt + 1 < nk) store_lds(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds column n = l32 of each 32x32 tile and 16 rows (mfma_row).
#pragma unroll
  for (int b = 0; b < TN; ++b) {
    const int64_t n = n0 + wn * WTN + b * 32 + l32;
    if (n >= p.N) continue;
    const float bias_n = p.bias ? p.bias[n] : 0.f;
    float sw_n = 0.f;
    if constexpr (INT8) sw_n = p.s_w[n];
#pragma unroll
    for (int a = 0; a < TM; ++a) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t m = m0 + wm * WTM + a * 32 + mfma_row(i, lane);
        if (m >= p.M) continue;
        const bool valid = p.row_valid == nullptr || p.row_valid[m] != 0;
        if constexpr (INT8) {
          const int32_t raw = acc[a][b][i];
          if (p.acc_out) p.acc_out[m * p.N + n] = raw;
          if (p.C) {
            // y = fp32(acc) * (s_a * s_w) + b, each operation rounded separately (no FMA).
            float v = static_cast<float>(raw) * (p.s_a[m] * sw_n);
            if (p.bias) v = v + bias_n;
            if (!valid) v = 0.f;
            store_out<TO>(p.C, m * p.ldc + n, v);
          }
        } else {
          float v = acc[a][b][i] + bias_n;
          if (!valid) v = 0.f;
          store_out<TO>(p.C, m * p.ldc + n, v);
        }
      }
    }
  }
}

template <typename T, typename TO, int BM, int BN, int WM, int WN, bool INT8>
int launch_gemm(const GemmArgs& a, hipStream_t stream) {
  const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  if (tiles <= 0) return MI355_OK;
  if (tiles > 0x7fffffffLL) return MI355_E_BAD_SIZE;
  hipLaunchKernelGGL((gemm_kernel<T, TO, BM, BN, WM, WN, INT8>), dim3(static_cast<unsigned>(tiles)),
                     dim3(WM * WN * 64), 0, stream, a);
  return static_cast<int>(hipGetLastError());
}

}  // namespace

template <typename T, int BM, int BN, int WM, int WN, bool INT8>
int launch_by_out(const GemmArgs& a, hipStream_t s) {
  switch (a.out_dtype) {
    case MI355_F16: return launch_gemm<T, _Float16, BM, BN, WM, WN, INT8>(a, s);
    case MI355_BF16: return launch_gemm<T, __bf16, BM, BN, WM, WN, INT8>(a, s);
    default: return launch_gemm<T, float, BM, BN, WM, WN, INT8>(a, s);
  }
}

extern "C" int mi355_gemm_bias(int in_dtype, int out_dtype, const void* A, int64_t lda,
                               const void* W, int64_t ldw, const float* bias, void* C, int64_t ldc,
                               int64_t M, int64_t N, int64_t K, const uint8_t* row_valid,
                               void* stream) {
  if (M < 0 || N < 0 || K < 0) return MI355_E_BAD_SIZE;
  if (M == 0 || N == 0) return MI355_OK;
  if (!A || !W || !C) return MI355_E_NULL_POINTER;
  const bool ok_in = in_dtype == MI355_F32 || in_dtype == MI355_F16 || in_dtype == MI355_BF16;
  const bool ok_out = out_dtype == MI355_F32 || out_dtype == MI355_F16 || out_dtype == MI355_BF16;
  if (!ok_in || !ok_out) return MI355_E_BAD_DTYPE;
  if ((in_dtype == MI355_F32) != (out_dtype == MI355_F32)) return MI355_E_UNSUPPORTED;
  const int64_t epc = in_dtype == MI355_F32 ? 4 : 8;
  if (K % epc || lda % epc || ldw % epc || !aligned16(A) || !aligned16(W))
    return MI355_E_ALIGNMENT;
  if (lda < K || ldw < K || ldc < N) return MI355_E_BAD_SIZE;
  GemmArgs a{};
  a.A = A;
  a.W = W;
  a.bias = bias;
  a.C = C;
  a.row_valid = row_valid;
  a.lda = lda;
  a.ldw = ldw;
  a.ldc = ldc;
  a.M = M;
  a.N = N;
  a.K = K;
  a.out_dtype = out_dtype;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (in_dtype) {
    case MI355_F16: return launch_by_out<_Float16, 256, 128, 2, 2, false>(a, s);
    case MI355_BF16: return launch_by_out<__bf16, 256, 128, 2, 2, false>(a, s);
    default: return launch_gemm<float, float, 128, 128, 2, 2, false>(a, s);
  }
}

extern "C" int mi355_gemm_i8(const int8_t* A, const int8_t* W, const float* s_a, const float* s_w,
                             const float* bias, int out_dtype, void* C, int64_t ldc,
                             int32_t* acc_out, int64_t M, int64_t N, int64_t K,
                             const uint8_t* row_valid, void* stream) {
  if (M < 0 || N < 0 || K < 0) return MI355_E_BAD_SIZE;
  if (M == 0 || N == 0) return MI355_OK;
  if (!A || !W || (!C && !acc_out)) return MI355_E_NULL_POINTER;
  if (C && (!s_a || !s_w)) return MI355_E_NULL_POINTER;
  if (out_dtype != MI355_F32 && out_dtype != MI355_F16 && out_dtype != MI355_BF16)
    return MI355_E_BAD_DTYPE;
  if (K % 16 || !aligned16(A) || !aligned16(W)) return MI355_E_ALIGNMENT;
  if (C && ldc < N) return MI355_E_BAD_SIZE;
  GemmArgs a{};
  a.A = A;
  a.W = W;
  a.bias = bias;
  a.C = C;
  a.acc_out = acc_out;
  a.s_a = s_a;
  a.s_w = s_w;
  a.row_valid = row_valid;
  a.lda = K;
  a.ldw = K;
  a.ldc = ldc;
  a.M = M;
  a.N = N;
  a.K = K;
  a.out_dtype = out_dtype;
  return launch_by_out<int8_t, 256, 128, 2, 2, true>(a, static_cast<hipStream_t>(stream));
}
