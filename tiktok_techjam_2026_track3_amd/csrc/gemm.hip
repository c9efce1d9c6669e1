// Projection GEMMs of the attention block on gfx950 MFMA:
//   C[M,N] = A[M,K] · W[N,K]^T + bias[N]                      (fp16 / bf16 / fp32, fp32 accumulate)
//   C[M,N] = fp32(A_i8 · W_i8^T) * (s_a[m] * s_w[n]) + bias[n] (int8 x int8 -> exact int32)
// Both operands are K-major (nn.Linear weight layout), so every MFMA fragment is one 16-byte LDS
// read per lane. Work-group tile BM x BN, waves arranged WM x WN, each wave owning
// (BM/WM) x (BN/WN) as 32x32 MFMA tiles. K is staged 128 bytes per row per step (64 fp16,
// 128 int8, 32 fp32 elements), double-buffered in LDS with an XOR swizzle on 16-byte chunks.
// The MFMA computes C^T blocks so each lane holds runs of 4 consecutive output features; the
// epilogue stages the finished tile in LDS and writes it back in 16-byte row chunks.
#include "common.h"

#include <mutex>

// interleave the LDS fragment reads of k-slice j+1 with the MFMAs of slice j: 1 = scheduler
// hints, 2 = explicit issue order (MFMA, read, MFMA, read, ... fenced by sched_barrier);
// measured on the projection shapes: 2 is 3-5% faster than 1
#ifndef MI355_GEMM_SCHED
#define MI355_GEMM_SCHED 2
#endif
// with the explicit issue order: alternate the issue priority of the two waves of a SIMD
// (1: per half K step, 2: per k-slice). Without it the older wave of each SIMD finishes its
// step's MFMAs ~1000 cycles before the younger one, which then runs alone on the MFMA pipe.
#ifndef MI355_GEMM_PP
#define MI355_GEMM_PP 1
#endif
// with the explicit issue order: spread each step's LDS-DMA loads over its MFMAs
#ifndef MI355_GEMM_SPREAD
#define MI355_GEMM_SPREAD 1
#endif

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
  const void* R;  // residual [M, N] of the output dtype, nullable: C = R + round(A W^T + b)
  const float* ln_stats;   // LayerNorm fold: per row (mean, rstd) [M][2] (LNF instances only)
  const float* ln_colsum;  // LayerNorm fold: per column sum_k W[n, k] of the folded weight
  int64_t lda, ldw, ldc, ldr;
  int64_t M, N, K;
  int out_dtype;
  int epi;  // EPI_* flags
  // Key-norm bounds of the attention that reads this projection's output (nullable; the
  // 256 x 256-tile instances with 16-bit outputs). The K block is columns [kb_col0, kb_col0 +
  // kb_heads * kb_hd), rows are kb_seq tokens per batch row: the tile of rows [m0, m0 + 256)
  // and the head's columns is key chunk (m0 % kb_seq) / 256 of batch row m0 / kb_seq, and its
  // bound max |k| is stored at kb_out[(b * kb_heads + h) * (kb_seq / 256) + chunk], with the
  // sign bit set when a row of the chunk has kb_valid 0 (the attention's bound pass format).
  float* kb_out;
  const uint8_t* kb_valid;
  int64_t kb_col0, kb_seq;
  int kb_hd, kb_heads;
};

// Epilogue options beyond bias / row mask / residual:
//   EPI_GELU         y = gelu(round(A W^T + b)): exact (erf) GELU in fp32 on the projection
//                    rounded to the output dtype, then rounded again (F.gelu on an nn.Linear
//                    output of that dtype); selects the GELU instantiation of the kernels;
//   EPI_ZERO_MASKED  rows whose row_valid entry is 0 are written as zeros after the residual
//                    add instead of as the residual (the block's trailing masked_fill).
constexpr int EPI_GELU = 1;
constexpr int EPI_ZERO_MASKED = 2;

// LayerNorm folded into the projection (compile-time variant LNF, mi355_layernorm_gemm_bias):
// A is the raw input x, W the weight with gamma folded in (W'[n, k] = W[n, k] gamma[k], rounded
// to the operand dtype), bias' = b + W beta, colsum[n] = sum_k W'[n, k]; with the row statistics
// (mean, rstd) of x the epilogue forms
//     y = rstd * (x W'^T - mean colsum) + bias' = ((x - mean) rstd gamma + beta) W^T + b,
// two FMAs per element. x W'^T accumulates exact products of the operands in fp32 and
// subtracting mean * colsum removes the row mean from the same rounded weights, so no
// cancellation beyond fp32 accumulation error is introduced.
MI355_DEVINL float ln_fold(float acc, float mean, float rstd, float colsum, float bias) {
  return __builtin_fmaf(rstd, __builtin_fmaf(-mean, colsum, acc), bias);
}

// Exact GELU, x * Phi(x) with Phi(x) = erfc(-x / sqrt 2) / 2, in fp32. erfc comes from the
// Chebyshev fit of Numerical Recipes (Press et al., "erfcc"; fractional error below 1.2e-7 for
// every argument):  erfc(z) = t exp(-z^2 - 1.26551223 + t P(t)),  t = 1 / (1 + z / 2),  z >= 0,
// with erfc(-z) = 2 - erfc(z) for the other sign. Branch-free (one reciprocal, one exponential,
// twelve FMAs): the epilogue evaluates it on every output of a 256 x 256 tile, where a
// general-purpose erff with range branches cost ~50% of the GEMM's time.
MI355_DEVINL float gelu_erf(float x) {
  const float z = __builtin_fabsf(x) * 0.70710678118654752f;
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.5f, z, 1.0f));
  float p = 0.17087277f;
  p = __builtin_fmaf(p, t, -0.82215223f);
  p = __builtin_fmaf(p, t, 1.48851587f);
  p = __builtin_fmaf(p, t, -1.13520398f);
  p = __builtin_fmaf(p, t, 0.27886807f);
  p = __builtin_fmaf(p, t, -0.18628806f);
  p = __builtin_fmaf(p, t, 0.09678418f);
  p = __builtin_fmaf(p, t, 0.37409196f);
  p = __builtin_fmaf(p, t, 1.00002368f);
  const float arg = __builtin_fmaf(t, p, __builtin_fmaf(-z, z, -1.26551223f));
  const float half_erfc = 0.5f * t * __builtin_amdgcn_exp2f(arg * 1.4426950408889634f);
  const float phi = x >= 0.f ? 1.0f - half_erfc : half_erfc;
  return x * phi;
}

template <typename TO>
MI355_DEVINL void store_out(void* C, int64_t idx, float v) {
  static_cast<TO*>(C)[idx] = from_f32<TO>(v);
}

constexpr int CH = 8;  // 16-byte chunks per LDS row per K step (128 bytes)

// Chunk swizzles (XOR of the 16-byte chunk index by row bits): conflict-free fragment reads
// (32 rows x one chunk per instruction) for 8-chunk (128-byte) and 4-chunk (64-byte) rows, checked
// against 32- and 64-bank LDS models.
MI355_DEVINL int swz8(int r) { return (r & 7) ^ ((r >> 3) & 1); }
template <int NCH>
MI355_DEVINL int swzc(int r) {
  if constexpr (NCH == 8)
    return swz8(r);
  else
    return ((r >> 1) & 3) ^ ((r >> 3) & 1);
}

// minimum waves per SIMD for work-groups of at most 4 waves (2: two work-groups share a CU)
#ifndef MI355_GEMM_WPE
#define MI355_GEMM_WPE 2
#endif

// direct (LDS-DMA) path: 16-byte chunks per row per K step, and depth of the LDS ring. Measured
// on the projection shapes: 8 chunks x 2 stages beats 4 chunks x 3-4 stages (the shorter K step
// doubles the barriers per tile)
#ifndef MI355_GEMM_CHD
#define MI355_GEMM_CHD 8
#endif
#ifndef MI355_GEMM_NST
#define MI355_GEMM_NST 2
#endif
// persistent tiles of one tile column whose K is one ring turn (N <= 256, K = 128 for 16-bit
// operands: the d_model-128 projections of the official shapes) keep W's stages in the ring
// and load only A after the first tile (1), or reload W with every tile (0)
#ifndef MI355_GEMM_WKEEP
#define MI355_GEMM_WKEEP 1
#endif

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

// DIRECT: K steps are fetched with buffer loads to LDS (64 lanes x 16 bytes land at
// M0 + 16*lane), so no registers or ds_write instructions carry the tiles, into a ring of NST
// slots of CHK chunks per row. Requires K % BK == 0. Otherwise a register-staged, double-
// buffered loader with bounds checks runs (8 chunks per row).
//
// PERSIST: the work-group loops over tiles pid = blockIdx.x, + gridDim.x, ... (grid = one work-group
// per CU). The last K step of a tile prefetches the next tile's first stage into the free ring
// slot, and the epilogue stores straight from registers (no LDS staging), so the next tile's loads
// and the previous tile's stores are in flight while MFMAs run. Requires DIRECT, K a multiple of
// NST steps, and 16-byte aligned output (and residual) rows whose feature count is a multiple of
// 8 (16-bit) or 4 (fp32).
template <typename T, typename TO, int BM, int BN, int WM, int WN, bool INT8, bool DIRECT, bool GELU,
          bool LNF, bool PERSIST = false>
__global__ __launch_bounds__(WM* WN * 64, (WM * WN <= 4) ? MI355_GEMM_WPE : 1) void gemm_kernel(GemmArgs p) {
  static_assert(!PERSIST || (DIRECT && !INT8), "persistent tiles: direct loads, 16-bit / fp32 operands");
  using MF = Mfma<T>;
  using frag = typename MF::frag;
  using acc_t = typename MF::acc;
  constexpr int NT = WM * WN * 64;
  constexpr int EPC = MF::ELEMS_PER_CHUNK;
  constexpr int CHK = DIRECT ? MI355_GEMM_CHD : CH;  // 16-byte chunks per row per K step
  constexpr int NST = DIRECT ? MI355_GEMM_NST : 2;   // LDS ring depth
  static_assert(CHK == 4 || CHK == 8, "chunks per row");
  constexpr int BK = CHK * EPC;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int A_LOADS = BM * CH / NT, B_LOADS = BN * CH / NT;
  static_assert((BM * CH) % NT == 0 && (BN * CH) % NT == 0, "loader shape");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
  // Output tile staged in LDS for coalesced 16-byte stores (row pitch padded by 16 bytes).
  constexpr int C_PITCH = BN * static_cast<int>(sizeof(TO)) + 16;
  constexpr int STAGE_BYTES = NST * (BM + BN) * CHK * 16;
  constexpr bool STAGE_C = BM * C_PITCH <= 160 * 1024 - 1024;
  // the key-norm bound epilogue (GemmArgs::kb_out): staged 256 x 256 tiles of 16-bit outputs
  constexpr bool KB_EPI = STAGE_C && BM == 256 && BN == 256 && sizeof(TO) == 2 && !INT8 &&
                          !PERSIST && WM * WN == 8;
  constexpr int LDS_BYTES = (STAGE_C && BM * C_PITCH > STAGE_BYTES) ? BM * C_PITCH : STAGE_BYTES;

  __shared__ u32x4 lds_raw[LDS_BYTES / 16];
  u32x4 (*lds)[(BM + BN) * CHK] = reinterpret_cast<u32x4 (*)[(BM + BN) * CHK]>(lds_raw);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t ntm = (p.M + BM - 1) / BM, ntn = (p.N + BN - 1) / BN;
  int64_t pid = blockIdx.x;
  int64_t m0, n0;
  auto tile_origin = [&](int64_t id, int64_t& tm0, int64_t& tn0) {
    int64_t tmi, tni;
    tile_coords(id, ntm, ntn, tmi, tni);
    tm0 = tmi * BM;
    tn0 = tni * BN;
  };
  tile_origin(pid, m0, n0);

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

  // acc[a][b] holds the 32x32 block (features wn*WTN + 32b .., tokens wm*WTM + 32a ..) as
  // D = W_rows . A_rows^T: lane l keeps token l%32 and features mfma_row(i, l).
  acc_t acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0;

  // direct loads (buffer loads to LDS): wave w issues blocks w, w + NW, ... of 8 rows (1 KB);
  // lane = (row r, physical chunk pc) fetches the logical chunk the swizzle places there. Each
  // lane's byte offset is fixed across K steps and the step advances the scalar offset; the
  // A / W resources start at the tile's first row and end at row M / N, so rows past the end
  // read as zeros (their results are never stored).
  constexpr int NWAVE = WM * WN;
  constexpr int RBK = 64 / CHK;            // rows per 1 KB block
  constexpr int BLOCKS = (BM + BN) / RBK;
  constexpr int NLD = BLOCKS / NWAVE;      // loads per wave per K step
  static_assert(BLOCKS % NWAVE == 0 && (BM / RBK) % NWAVE == 0, "direct loader shape");
  static_assert(BM % 16 == 0, "B rows keep the swizzle phase of their stage row");
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t a_pitch = static_cast<uint32_t>(p.lda) * ES, w_pitch = static_cast<uint32_t>(p.ldw) * ES;
  // buffer resources of the tile at (tm0, tn0): its A rows and W rows, ranges ending at M / N
  auto tile_rsrc = [&](int64_t tm0, int64_t tn0, u32x4& ar, u32x4& wr) {
    const uint32_t a_bytes = static_cast<uint32_t>(p.M - tm0 < BM ? p.M - tm0 : BM) * a_pitch;
    const uint32_t w_bytes = static_cast<uint32_t>(p.N - tn0 < BN ? p.N - tn0 : BN) * w_pitch;
    ar = buffer_rsrc(Ab + tm0 * static_cast<int64_t>(a_pitch), a_bytes);
    wr = buffer_rsrc(Wb + tn0 * static_cast<int64_t>(w_pitch), w_bytes);
  };
  uint32_t doff[NLD];
#pragma unroll
  for (int i = 0; i < NLD; ++i) {
    const int row = (wv + i * NWAVE) * RBK + lane / CHK;  // row within the A|B stage
    const int c = (lane % CHK) ^ swzc<CHK>(row);
    doff[i] = row < BM ? static_cast<uint32_t>(row) * a_pitch + c * 16u
                       : static_cast<uint32_t>(row - BM) * w_pitch + c * 16u;
  }
  // issued from inline assembly (buffer_dma_lds16): the compiler then keeps precise LDS wait
  // counts for the fragment reads instead of draining every outstanding load before each one
  // this tile's resources and (PERSIST) the next tile's, whose first stage the last K step loads
  u32x4 a_rsrc, w_rsrc, na_rsrc, nw_rsrc;
  tile_rsrc(m0, n0, a_rsrc, w_rsrc);
  // PERSIST with one column of tiles and K of exactly one ring turn (N <= BN, nk == NST): every
  // tile's W stages are the same bytes in the same slots (nothing else writes the ring), so after
  // the first tile only A is loaded (w_held; MI355_GEMM_WKEEP)
  bool w_held = false;
  auto load_one = [&](int s, int64_t k0, int i, bool nxt) {
    const uint32_t so = static_cast<uint32_t>(k0) * ES;
    const int blk = wv + i * NWAVE;
    if (i < (BM / RBK) / NWAVE)
      buffer_dma_lds16(nxt ? na_rsrc : a_rsrc, doff[i], so, lds_addr_of(&lds[s][blk * 64]));
    else if (!(PERSIST && MI355_GEMM_WKEEP && w_held))
      buffer_dma_lds16(nxt ? nw_rsrc : w_rsrc, doff[i], so, lds_addr_of(&lds[s][blk * 64]));
  };
  auto load_direct = [&](int s, int64_t k0, bool nxt = false) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) load_one(s, k0, i, nxt);
  };

  const int nk = static_cast<int>((p.K + BK - 1) / BK);
  const int g = lane >> 5, l32 = lane & 31;

  // MFMAs of one K step from ring slot `cur`; the fragments of k-slice j+1 are read while the
  // MFMAs of slice j run (two register sets)
  // dma_slot >= 0: the NLD loads of K offset dma_k0 into that ring slot are issued between the
  // MFMAs of the first half of the step (one after every DMA_EVERY-th MFMA), so the work-group's
  // loads do not reach the memory system as one burst after the barrier
  constexpr int DMA_EVERY = (TM * TN * (CHK / 2)) / (2 * NLD) > 0 ? (TM * TN * (CHK / 2)) / (2 * NLD) : 1;
  static_assert(NLD * DMA_EVERY <= TM * TN * (CHK / 2), "every load of a step has an MFMA slot");
  auto compute = [&](const int cur, const int dma_slot = -1, const int64_t dma_k0 = 0, const bool dma_next = false) {
    frag fa[2][TM], fb[2][TN];
    auto read_frag = [&](int j, int buf, int f) {
      const int c = 2 * j + g;
      if (f < TM) {
        const int row = wm * WTM + f * 32 + l32;
        fa[buf][f] = __builtin_bit_cast(frag, lds[cur][row * CHK + (c ^ swzc<CHK>(row))]);
      } else {
        const int row = wn * WTN + (f - TM) * 32 + l32;
        fb[buf][f - TM] = __builtin_bit_cast(frag, lds[cur][(BM + row) * CHK + (c ^ swzc<CHK>(row))]);
      }
    };
#pragma unroll
    for (int f = 0; f < TM + TN; ++f) read_frag(0, 0, f);
#pragma unroll
    for (int j = 0; j < CHK / 2; ++j) {
#if MI355_GEMM_SCHED == 2
      // explicit issue order: MFMA i of slice j, then fragment i of slice j+1 (sched_barrier
      // fences keep the compiler from pairing each read with the MFMA that consumes it)
#if MI355_GEMM_PP
      {
        // the two waves sharing a SIMD (w and w + NWAVE/2) take turns at the higher issue
        // priority, so neither runs far ahead and leaves the other alone on the MFMA pipe
        const int half = MI355_GEMM_PP == 1 ? (j >= CHK / 4) : (j & 1);
        if ((wv >= NWAVE / 2) != (half != 0))
          __builtin_amdgcn_s_setprio(1);
        else
          __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
      }
#endif
      // (a wave tile of one MFMA block has more fragments per slice than MFMAs: the loop runs
      // to the larger count, issuing MFMAs only for the first TM * TN positions)
      constexpr int NPOS = TM * TN > TM + TN ? TM * TN : TM + TN;
#pragma unroll
      for (int i = 0; i < NPOS; ++i) {
        if (i < TM * TN) {
          const int a = i / TN, b = i % TN;
          acc[a][b] = MF::mma(fb[j & 1][b], fa[j & 1][a], acc[a][b]);
          __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (DIRECT) {
          const int q = j * TM * TN + i;  // MFMA index within the step
          if (i < TM * TN && dma_slot >= 0 && q % DMA_EVERY == DMA_EVERY - 1 && q / DMA_EVERY < NLD) {
            load_one(dma_slot, dma_k0, q / DMA_EVERY, dma_next);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        if (j + 1 < CHK / 2 && i < TM + TN) {
          read_frag(j + 1, (j + 1) & 1, i);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
#else
      if (j + 1 < CHK / 2) {
#pragma unroll
        for (int f = 0; f < TM + TN; ++f) read_frag(j + 1, (j + 1) & 1, f);
      }
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = MF::mma(fb[j & 1][b], fa[j & 1][a], acc[a][b]);
#if MI355_GEMM_SCHED
      // issue order: MFMA, LDS read, MFMA, LDS read, ... then the remaining MFMAs
      if (j + 1 < CHK / 2) {
#pragma unroll
        for (int i = 0; i < TM + TN; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, TM * TN - (TM + TN), 0);
      }
#endif
#endif
    }
  };

  const bool col_vec = ((reinterpret_cast<uintptr_t>(p.bias) | reinterpret_cast<uintptr_t>(p.s_w) |
                         reinterpret_cast<uintptr_t>(p.ln_colsum)) & 15u) == 0;
  auto col4 = [&](const float* arr, int64_t nb) MI355_LAMBDA_INLINE {
    f32x4 r = {0.f, 0.f, 0.f, 0.f};
    if (arr == nullptr) return r;
    if (col_vec && nb + 3 < p.N) return *reinterpret_cast<const f32x4*>(arr + nb);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (nb + e < p.N) r[e] = arr[nb + e];
    return r;
  };

  // PERSIST epilogue: the values of the staged epilogue below (bias or folded LayerNorm, GELU,
  // row mask, one rounding to TO, residual, zeroed rows), stored from registers. Lane (l32, g)
  // holds features 8 i4 + 4 g .. + 3 of token l32 (i4 = 0..3). fp32 outputs store each group of
  // 4 as 16 bytes; 16-bit outputs pack groups i4 = 2j and 2j + 1 and swap them across the lane
  // pair (l, l + 32) with v_permlane32_swap, after which lane g holds features 16 j + 8 g .. + 7:
  // one 16-byte store. The host guarantees 16-byte aligned rows and N a multiple of 16 / sizeof(TO).
  auto epilogue_direct = [&]() MI355_LAMBDA_INLINE {
    constexpr int EPC_OUT = 16 / static_cast<int>(sizeof(TO));
    bool in_m[TM], valid[TM];
    float mean[TM], rstd[TM];
#pragma unroll
    for (int a = 0; a < TM; ++a) {
      const int64_t m = m0 + wm * WTM + a * 32 + l32;
      in_m[a] = m < p.M;
      valid[a] = !in_m[a] || p.row_valid == nullptr || p.row_valid[m] != 0;
      mean[a] = 0.f;
      rstd[a] = 0.f;
      if constexpr (LNF) {
        if (in_m[a]) {
          mean[a] = p.ln_stats[2 * m];
          rstd[a] = p.ln_stats[2 * m + 1];
        }
      }
    }
    // the projection value of element e of group i4 for row block a, rounded to TO
    auto value = [&](int a, int b, int i4, int e, const f32x4& bias4, const f32x4& cs4) MI355_LAMBDA_INLINE {
      float v;
      if constexpr (LNF)
        v = ln_fold(acc[a][b][4 * i4 + e], mean[a], rstd[a], cs4[e], bias4[e]);
      else
        v = acc[a][b][4 * i4 + e] + bias4[e];
      if constexpr (GELU) v = gelu_erf(to_f32(from_f32<TO>(v)));
      if (!valid[a]) v = 0.f;
      return from_f32<TO>(v);
    };
    // residual add on the rounded projection (rc: the residual chunk, read before any write of
    // the block: R may be C), zeroed rows
    auto finish = [&](u32x4 chunk, int64_t m, int64_t n, bool ok, const u32x4& rc) MI355_LAMBDA_INLINE {
      if (p.R) {
        TO* cv = reinterpret_cast<TO*>(&chunk);
        const TO* rv = reinterpret_cast<const TO*>(&rc);
#pragma unroll
        for (int e = 0; e < EPC_OUT; ++e) cv[e] = from_f32<TO>(to_f32(cv[e]) + to_f32(rv[e]));
      }
      if (!ok && (p.epi & EPI_ZERO_MASKED)) chunk = u32x4{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(static_cast<TO*>(p.C) + m * p.ldc + n) = chunk;
    };
    // Residual chunks are requested two at a time before the stores that use them (16-bit
    // outputs: the TM (<= 2) row blocks of a (b, j); fp32 outputs: the two halves h of an
    // (a, b, j)).
    // One at a time, each load waited for behind the previous store, the residual had doubled the
    // epilogue's time (official shape 6's fp32 out projection 0.31 -> 0.59 ms).
    static_assert(TM <= 2, "at most two residual chunks per batch");
    auto res_load = [&](u32x4& r, int64_t m, int64_t n, bool in) MI355_LAMBDA_INLINE {
      r = u32x4{0u, 0u, 0u, 0u};
      if (p.R && in) r = *reinterpret_cast<const u32x4*>(static_cast<const TO*>(p.R) + m * p.ldr + n);
    };
#pragma unroll
    for (int b = 0; b < TN; ++b) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        u32x4 rres[2];
        if constexpr (sizeof(TO) == 2) {
          const int64_t n = n0 + wn * WTN + b * 32 + 16 * j + 8 * g;
#pragma unroll
          for (int a = 0; a < TM; ++a)
            res_load(rres[a], m0 + wm * WTM + a * 32 + l32, n, in_m[a] && n < p.N);
        }
        const int64_t nb = n0 + wn * WTN + b * 32 + 16 * j + 4 * g;  // group i4 = 2j; 2j + 1 at +8
        const f32x4 bias0 = col4(p.bias, nb), bias1 = col4(p.bias, nb + 8);
        const f32x4 cs0 = LNF ? col4(p.ln_colsum, nb) : f32x4{0.f, 0.f, 0.f, 0.f};
        const f32x4 cs1 = LNF ? col4(p.ln_colsum, nb + 8) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int a = 0; a < TM; ++a) {
          const int64_t m = m0 + wm * WTM + a * 32 + l32;
          if constexpr (sizeof(TO) == 4) {
#pragma unroll
            for (int h = 0; h < 2; ++h) res_load(rres[h], m, nb + 8 * h, in_m[a] && nb + 8 * h < p.N);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              f32x4 w;
#pragma unroll
              for (int e = 0; e < 4; ++e)
                w[e] = value(a, b, 2 * j + h, e, h ? bias1 : bias0, h ? cs1 : cs0);
              if (in_m[a] && nb + 8 * h < p.N)
                finish(__builtin_bit_cast(u32x4, w), m, nb + 8 * h, valid[a], rres[h]);
            }
          } else {
            typedef TO to2 __attribute__((ext_vector_type(2)));
            uint32_t lo[2], hi[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const f32x4& bb = h ? bias1 : bias0;
              const f32x4& cc = h ? cs1 : cs0;
              lo[h] = __builtin_bit_cast(uint32_t, to2{value(a, b, 2 * j + h, 0, bb, cc), value(a, b, 2 * j + h, 1, bb, cc)});
              hi[h] = __builtin_bit_cast(uint32_t, to2{value(a, b, 2 * j + h, 2, bb, cc), value(a, b, 2 * j + h, 3, bb, cc)});
            }
            // every lane takes part in the swaps, stored or not
            const auto rl = __builtin_amdgcn_permlane32_swap(lo[0], lo[1], false, false);
            const auto rh = __builtin_amdgcn_permlane32_swap(hi[0], hi[1], false, false);
            const u32x4 chunk = {rl[0], rh[0], rl[1], rh[1]};
            const int64_t n = n0 + wn * WTN + b * 32 + 16 * j + 8 * g;
            if (in_m[a] && n < p.N) finish(chunk, m, n, valid[a], rres[a]);
          }
        }
      }
    }
  };

  if constexpr (DIRECT) {
    // ring of NST slots: step kt computes slot kt % NST while steps kt+1 .. kt+NST-1 are in
    // flight; before the barrier a wave waits only for its loads of step kt+1
    constexpr int VM_FULL = (NST - 2) * NLD;  // loads issued after those of step kt+1
    static_assert(VM_FULL < 64, "vmcnt range");
    // s_waitcnt immediate: vmcnt(VM_FULL), lgkmcnt(0) (no LDS read of the slot refilled next may
    // still be in flight), expcnt not waited
    constexpr int WAIT_FULL = (VM_FULL & 15) | ((VM_FULL >> 4) << 14) | (7 << 4);
    // Work-group barrier without __syncthreads()'s release fence, which would wait for every
    // outstanding LDS-DMA load and so drain the ring; the explicit s_waitcnt before it provides
    // exactly the ordering needed, and the empty asm statements keep the compiler from moving
    // memory operations across it.
    auto ring_barrier = [] {
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    };
#pragma unroll
    for (int st = 0; st < NST - 1; ++st)
      if (st < nk) load_direct(st, static_cast<int64_t>(st) * BK);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // PERSIST: another tile follows. Steps kl >= nk then load that tile's steps kl - nk, which
    // land in the slots its own steps compute from because nk is a multiple of NST. With NST = 2
    // the step-end wait is vmcnt(0), which also covers the previous epilogue's stores whatever
    // order loads and stores complete in.
    bool has_next = false;
    auto step = [&](const int kt, const int slot) {
      const int kl = kt + NST - 1;
      const bool nxt = PERSIST && kl >= nk && has_next;
      const bool load = kl < nk || nxt;
      const int64_t lk0 = static_cast<int64_t>(kl < nk ? kl : kl - nk) * BK;
#if MI355_GEMM_SCHED == 2 && MI355_GEMM_SPREAD
      compute(slot, load ? (slot + NST - 1) % NST : -1, lk0, nxt);
#else
      if (load) load_direct((slot + NST - 1) % NST, lk0, nxt);
      compute(slot);
#endif
      if (load)
        __builtin_amdgcn_s_waitcnt(WAIT_FULL);
      else
        __builtin_amdgcn_s_waitcnt(0);
      ring_barrier();
    };
    auto k_loop = [&]() MI355_LAMBDA_INLINE {
      int kt = 0;
      for (; kt + NST <= nk; kt += NST) {
#pragma unroll
        for (int u = 0; u < NST; ++u) step(kt + u, u);
      }
#pragma unroll
      for (int u = 0; u < NST - 1; ++u)
        if (kt + u < nk) step(kt + u, u);
    };
    if constexpr (PERSIST) {
      const bool w_keep = MI355_GEMM_WKEEP && ntn == 1 && nk == NST;
      for (;;) {
        const int64_t npid = pid + gridDim.x;
        has_next = npid < ntm * ntn;
        int64_t nm0 = 0, nn0 = 0;
        if (has_next) {
          tile_origin(npid, nm0, nn0);
          tile_rsrc(nm0, nn0, na_rsrc, nw_rsrc);
        }
        k_loop();
        // from here on every W load would rewrite the bytes the slots hold (see w_held)
        w_held = w_keep;
        epilogue_direct();
        if (!has_next) return;
        pid = npid;
        m0 = nm0;
        n0 = nn0;
        a_rsrc = na_rsrc;
        w_rsrc = nw_rsrc;
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
          for (int b = 0; b < TN; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[a][b][i] = 0;
      }
    } else {
      k_loop();
    }
  } else {
    load_global(0);
    store_lds(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load_global(static_cast<int64_t>(kt + 1) * BK);
      compute(cur);
      if (kt + 1 < nk) store_lds(cur ^ 1);
      __syncthreads();
    }
  }

  // ---- epilogue: per element bias / dequantisation / row mask, rounded once to TO
  // Per-row values (row mask, int8 activation scale, LayerNorm statistics) are read once per row;
  // per-column values (bias, int8 weight scale, folded-LayerNorm column sums) once per group of
  // 4 consecutive features, as one 16-byte load when the group is inside N and the arrays are
  // 16-byte aligned, and shared by the TM row blocks.
  char* cl = reinterpret_cast<char*>(lds_raw);
  // a tile of the K block whose key-norm bounds this epilogue writes (see the end); its key-mask
  // bytes are requested here, long before they are needed
  bool kb_tile = false;
  int kb_bad = 0;
  if constexpr (KB_EPI) {
    kb_tile = p.kb_out != nullptr && n0 >= p.kb_col0 &&
              n0 < p.kb_col0 + static_cast<int64_t>(p.kb_heads) * p.kb_hd;
    if (kb_tile && tid < BM && p.kb_valid != nullptr) kb_bad = p.kb_valid[m0 + tid] == 0;
  }
  bool in_m_[TM], valid_[TM];
  float sa_m[TM], mean_m[TM], rstd_m[TM];
#pragma unroll
  for (int a = 0; a < TM; ++a) {
    const int64_t m = m0 + wm * WTM + a * 32 + l32;
    in_m_[a] = m < p.M;
    valid_[a] = !in_m_[a] || p.row_valid == nullptr || p.row_valid[m] != 0;
    sa_m[a] = 0.f;
    if constexpr (INT8) sa_m[a] = in_m_[a] ? p.s_a[m] : 0.f;
    mean_m[a] = 0.f;
    rstd_m[a] = 0.f;
    if constexpr (LNF) {
      if (in_m_[a]) {
        mean_m[a] = p.ln_stats[2 * m];
        rstd_m[a] = p.ln_stats[2 * m + 1];
      }
    }
  }
#pragma unroll
  for (int b = 0; b < TN; ++b) {
    // a 32-feature block entirely past N: its staged values are never copied out (wave-uniform)
    if (n0 + wn * WTN + b * 32 >= p.N) continue;
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int n_loc = wn * WTN + b * 32 + 8 * i4 + 4 * g;  // 4 consecutive features
      const int64_t nb = n0 + n_loc;
      const f32x4 bias4 = col4(p.bias, nb);
      const f32x4 sw4 = INT8 ? col4(p.s_w, nb) : f32x4{0.f, 0.f, 0.f, 0.f};
      const f32x4 cs4 = LNF ? col4(p.ln_colsum, nb) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int a = 0; a < TM; ++a) {
        const int m_loc = wm * WTM + a * 32 + l32;
        const int64_t m = m0 + m_loc;
        const bool in_m = in_m_[a];
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t n = nb + e;
          const bool in_n = n < p.N;
          const float bias_n = bias4[e];
          if constexpr (INT8) {
            const int32_t raw = acc[a][b][4 * i4 + e];
            if (p.acc_out && in_m && in_n) p.acc_out[m * p.N + n] = raw;
            // y = fp32(acc) * (s_a * s_w) + b, each operation rounded separately (no FMA).
            float y = static_cast<float>(raw) * (sa_m[a] * sw4[e]);
            if (p.bias) y = y + bias_n;
            v[e] = y;
          } else if constexpr (LNF) {
            v[e] = ln_fold(acc[a][b][4 * i4 + e], mean_m[a], rstd_m[a], cs4[e], bias_n);
          } else {
            v[e] = acc[a][b][4 * i4 + e] + bias_n;
          }
          if constexpr (GELU) v[e] = gelu_erf(to_f32(from_f32<TO>(v[e])));
          if (!valid_[a]) v[e] = 0.f;
        }
        if constexpr (STAGE_C) {
          typedef TO to4 __attribute__((ext_vector_type(4)));
          to4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = from_f32<TO>(v[e]);
          *reinterpret_cast<to4*>(cl + m_loc * C_PITCH + n_loc * static_cast<int>(sizeof(TO))) = w;
        } else {
          if (p.C && in_m) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int64_t n = n0 + n_loc + e;
              if (n >= p.N) continue;
              float y = to_f32(from_f32<TO>(v[e]));  // the projection output, rounded once
              if (p.R) y = y + to_f32(static_cast<const TO*>(p.R)[m * p.ldr + n]);
              if (!valid_[a] && (p.epi & EPI_ZERO_MASKED)) y = 0.f;
              store_out<TO>(p.C, m * p.ldc + n, y);
            }
          }
        }
      }
    }
  }
  if constexpr (STAGE_C) {
    __syncthreads();
    if (p.C) {
      // coalesced copy of the staged tile: 16-byte chunks, rows of BN outputs
      constexpr int CPR = BN * static_cast<int>(sizeof(TO)) / 16;  // chunks per row
      constexpr int EPC_OUT = 16 / static_cast<int>(sizeof(TO));
      const bool vec_ok = (p.ldc % EPC_OUT) == 0 && ((reinterpret_cast<uintptr_t>(p.C) & 15u) == 0) &&
                          (!p.R || ((p.ldr % EPC_OUT) == 0 && (reinterpret_cast<uintptr_t>(p.R) & 15u) == 0));
      constexpr int PER = BM * CPR / NT;  // chunks per thread
      static_assert((BM * CPR) % NT == 0, "epilogue chunks");
      if (p.R && vec_ok) {
        // residual: every residual chunk of this thread is requested before the first is used,
        // so the loads' latency is paid once rather than once per chunk. Each chunk is read
        // before the same thread writes it, so R may be C.
        const TO* Rb = static_cast<const TO*>(p.R);
        u32x4 rc[PER];
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const int idx = tid + i * NT, r = idx / CPR, c = idx % CPR;
          const int64_t m = m0 + r, n = n0 + static_cast<int64_t>(c) * EPC_OUT;
          rc[i] = u32x4{0u, 0u, 0u, 0u};
          if (m < p.M && n + EPC_OUT <= p.N) rc[i] = *reinterpret_cast<const u32x4*>(Rb + m * p.ldr + n);
        }
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const int idx = tid + i * NT, r = idx / CPR, c = idx % CPR;
          const int64_t m = m0 + r, n = n0 + static_cast<int64_t>(c) * EPC_OUT;
          if (m >= p.M || n >= p.N) continue;
          u32x4 chunk = *reinterpret_cast<const u32x4*>(cl + r * C_PITCH + c * 16);
          TO* dst = static_cast<TO*>(p.C) + m * p.ldc + n;
          TO* cv = reinterpret_cast<TO*>(&chunk);
          const bool zero = (p.epi & EPI_ZERO_MASKED) && p.row_valid && p.row_valid[m] == 0;
          if (n + EPC_OUT <= p.N) {
            const TO* rv = reinterpret_cast<const TO*>(&rc[i]);
#pragma unroll
            for (int e = 0; e < EPC_OUT; ++e) cv[e] = from_f32<TO>(to_f32(cv[e]) + to_f32(rv[e]));
            if (zero) chunk = u32x4{0u, 0u, 0u, 0u};
            *reinterpret_cast<u32x4*>(dst) = chunk;
          } else {
            const TO* res = Rb + m * p.ldr + n;
            for (int e = 0; e < EPC_OUT && n + e < p.N; ++e)
              dst[e] = zero ? from_f32<TO>(0.f) : from_f32<TO>(to_f32(cv[e]) + to_f32(res[e]));
          }
        }
      } else
      for (int idx = tid; idx < BM * CPR; idx += NT) {
        const int r = idx / CPR, c = idx % CPR;
        const int64_t m = m0 + r, n = n0 + static_cast<int64_t>(c) * EPC_OUT;
        if (m >= p.M || n >= p.N) continue;
        u32x4 chunk = *reinterpret_cast<const u32x4*>(cl + r * C_PITCH + c * 16);
        TO* dst = static_cast<TO*>(p.C) + m * p.ldc + n;
        const bool zero = (p.epi & EPI_ZERO_MASKED) && p.row_valid && p.row_valid[m] == 0;
        const TO* res = (p.R && !zero) ? static_cast<const TO*>(p.R) + m * p.ldr + n : nullptr;
        if (vec_ok && n + EPC_OUT <= p.N) {
          if (res) {
            // residual add on the rounded projection output (the reference adds two tensors of
            // the output dtype); read before the write, so R may be C itself
            const u32x4 rc = *reinterpret_cast<const u32x4*>(res);
            TO* cv = reinterpret_cast<TO*>(&chunk);
            const TO* rv = reinterpret_cast<const TO*>(&rc);
#pragma unroll
            for (int e = 0; e < EPC_OUT; ++e) cv[e] = from_f32<TO>(to_f32(cv[e]) + to_f32(rv[e]));
          }
          *reinterpret_cast<u32x4*>(dst) = chunk;
        } else {
          const TO* src = reinterpret_cast<const TO*>(&chunk);
          for (int e = 0; e < EPC_OUT && n + e < p.N; ++e)
            dst[e] = res ? from_f32<TO>(to_f32(src[e]) + to_f32(res[e])) : src[e];
        }
      }
    }
    if constexpr (KB_EPI) {
      // A tile of the K block (GemmArgs::kb_out): the key-norm bounds of its BN / kb_hd heads
      // over its 256 rows, from the staged tile (which the copy above only read). Each thread
      // takes one head and BM / (threads per head) rows; a key's |k|^2 is chunk_sq over its
      // chunks combined by chunk_tree (the bound pass's bits); then maxima over the rows, the
      // waves of the head and, for the sign bit, the key mask of the 256 rows (loaded at the
      // start of the epilogue). The host guarantees whole tiles (M, kb_seq and kb_col0
      // multiples of 256) and an unmasked projection into 16-byte aligned rows.
      if (kb_tile) {
        using frag16 = typename Mfma<TO>::frag;
        auto bound_rows = [&](auto lk_c) MI355_LAMBDA_INLINE {
          constexpr int LK = decltype(lk_c)::value;     // 16-byte chunks per head row
          constexpr int TPH = NT / (BN / (8 * LK));     // threads per head
          const int hl = tid / TPH, t = tid % TPH;
          float m = 0.f;
#pragma unroll
          for (int r = t; r < BM; r += TPH) {
            float sq[LK];
#pragma unroll
            for (int j = 0; j < LK; ++j)
              sq[j] = chunk_sq(__builtin_bit_cast(
                  frag16, *reinterpret_cast<const u32x4*>(cl + r * C_PITCH + (hl * LK + j) * 16)));
            m = __builtin_elementwise_maximum(m, chunk_tree<LK>(sq));
          }
          return m;
        };
        const int lk = p.kb_hd / 8;
        float m = lk == 4 ? bound_rows(std::integral_constant<int, 4>{})
                : lk == 8 ? bound_rows(std::integral_constant<int, 8>{})
                          : bound_rows(std::integral_constant<int, 16>{});
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) m = __builtin_elementwise_maximum(m, __shfl_xor(m, off));
        __shared__ float kb_red[NT / 64];
        if (lane == 0) kb_red[wave] = m;
        const bool any_bad = __syncthreads_or(kb_bad) != 0;
        const int heads = BN / p.kb_hd, wph = (NT / 64) / heads;  // waves per head
        if (tid < heads) {
          float v = kb_red[tid * wph];
          for (int w = 1; w < wph; ++w) v = __builtin_elementwise_maximum(v, kb_red[tid * wph + w]);
          v = __builtin_fabsf(__builtin_sqrtf(v));
          const int64_t chunks = p.kb_seq / 256, bb = m0 / p.kb_seq, ci = (m0 % p.kb_seq) / 256;
          const int64_t hh = (n0 - p.kb_col0) / p.kb_hd + tid;
          p.kb_out[(bb * p.kb_heads + hh) * chunks + ci] = any_bad ? -v : v;
        }
      }
    }
  }
}

#ifndef MI355_GEMM_DIRECT
#define MI355_GEMM_DIRECT 1
#endif
#ifndef MI355_GEMM_NARROW
#define MI355_GEMM_NARROW 1
#endif
#ifndef MI355_GEMM_FILL
#define MI355_GEMM_FILL 256
#endif
#ifndef MI355_GEMM_FILL64
#define MI355_GEMM_FILL64 128
#endif
// fp32 operands: 64 x 64 tiles below this many 128 x 128 tiles (one per CU: official shape 11,
// whose fp32 projections are 8192 x 384 / 128 x 128, 0.45 -> 0.33 ms per forward against 64)
#ifndef MI355_GEMM_F32_FILL
#define MI355_GEMM_F32_FILL 256
#endif

// Small problems (at most 512 tiles of 32 x 32 outputs: the fp32 configuration's projections
// are 128 x 768 x 256 and 128 x 256 x 256; the official shapes' small batches), fp32 or 16-bit:
// a 32 x 32 output tile per work-group whose NWS waves split K. With one wave per tile the
// tile's MFMA chain (K/2 fp32 MFMAs, K/16 16-bit ones) runs in sequence; split NWS ways the
// chain is NWS times shorter and NWS times more SIMDs share it, where a 256 x 256 tile would
// leave all but a handful of CUs idle. Fragments come straight from
// global memory (lane (l32, g) reads 16 bytes of row l32 for chunk 2j + g; rows are K-major),
// U chunk pairs per wave requested before the first MFMA. The NWS partial tiles are summed
// through LDS in wave order (deterministic), then bias, row mask and residual are applied per
// element as in gemm_kernel's epilogue and the tile is written row by row.
template <typename T, int NWS, bool GELU, bool LNF, typename TO>
__global__ __launch_bounds__(64 * NWS) void gemm_splitk(GemmArgs p) {
  constexpr int U = 4;
  constexpr int PITCH = 65;  // padded: the reduction reads 32 features of one token per half-wave
  __shared__ float red[NWS][16][PITCH];
  using MF = Mfma<T>;
  using frag = typename MF::frag;
  constexpr int EPC = MF::ELEMS_PER_CHUNK;  // elements per 16-byte chunk
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int64_t ntm = (p.M + 31) / 32, ntn = (p.N + 31) / 32;
  int64_t tmi, tni;
  tile_coords(blockIdx.x, ntm, ntn, tmi, tni);
  const int64_t m0 = tmi * 32, n0 = tni * 32;
  const int64_t am = m0 + l32, wn = n0 + l32;
  const bool a_ok = am < p.M, w_ok = wn < p.N;
  const T* arow = static_cast<const T*>(p.A) + (a_ok ? am : 0) * p.lda;
  const T* wrow = static_cast<const T*>(p.W) + (w_ok ? wn : 0) * p.ldw;
  const int nchunk = static_cast<int>(p.K / EPC);

  // D = W_rows . A_rows^T: lane l keeps token l % 32 and features mfma_row(i, l)
  typename MF::acc acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
  // wave w takes chunk pairs w, w + NWS, w + 2 NWS, ...; half-wave g the pair's chunk g (A and W
  // take the same chunk in every lane, so the MFMA's k order inside a pair does not matter)
  for (int base = 2 * wave; base < nchunk; base += 2 * NWS * U) {
    frag fa[U], fw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = base + u * 2 * NWS + g;
      const bool in = c < nchunk;
      const u32x4 zero = {0u, 0u, 0u, 0u};
      fa[u] = __builtin_bit_cast(frag, (in && a_ok) ? *reinterpret_cast<const u32x4*>(arow + EPC * c) : zero);
      fw[u] = __builtin_bit_cast(frag, (in && w_ok) ? *reinterpret_cast<const u32x4*>(wrow + EPC * c) : zero);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc = MF::mma(fw[u], fa[u], acc);
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) red[wave][i][lane] = acc[i];
  __syncthreads();

  // element (token m_loc, feature n_loc) lives in register i of lane l: n_loc = mfma_row(i, l)
  for (int e = tid; e < 32 * 32; e += 64 * NWS) {
    const int n_loc = e & 31, m_loc = e >> 5;
    const int64_t m = m0 + m_loc, n = n0 + n_loc;
    if (m >= p.M || n >= p.N) continue;
    const int l = m_loc + 32 * ((n_loc >> 2) & 1), i = (n_loc >> 3) * 4 + (n_loc & 3);
    float v = red[0][i][l];
#pragma unroll
    for (int w = 1; w < NWS; ++w) v += red[w][i][l];
    if constexpr (LNF)
      v = ln_fold(v, p.ln_stats[2 * m], p.ln_stats[2 * m + 1], p.ln_colsum[n], p.bias ? p.bias[n] : 0.f);
    else if (p.bias)
      v = v + p.bias[n];
    // the projection rounded to the output type first (a no-op for fp32), as in gemm_kernel
    v = to_f32(from_f32<TO>(v));
    if constexpr (GELU) v = gelu_erf(v);
    const bool masked = p.row_valid && p.row_valid[m] == 0;
    if (masked) v = 0.f;
    // residual read before the write of the same element: R may be C
    if (p.R) v = to_f32(from_f32<TO>(v)) + to_f32(static_cast<const TO*>(p.R)[m * p.ldr + n]);
    if (masked && (p.epi & EPI_ZERO_MASKED)) v = 0.f;
    store_out<TO>(p.C, m * p.ldc + n, v);
  }
}

template <typename T, typename TO>
int launch_gemm_splitk(const GemmArgs& a, hipStream_t stream) {
  constexpr int NWS = 8;
  const int64_t tiles = ((a.M + 31) / 32) * ((a.N + 31) / 32);
  const dim3 grid(static_cast<unsigned>(tiles)), block(64 * NWS);
  // GELU is a compile-time variant: as a run-time option its inlined code in the unrolled
  // epilogue slowed every projection by ~10%
  const bool lnf = a.ln_stats != nullptr;
  if (a.epi & EPI_GELU) {
    if (lnf) hipLaunchKernelGGL((gemm_splitk<T, NWS, true, true, TO>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((gemm_splitk<T, NWS, true, false, TO>), grid, block, 0, stream, a);
  } else {
    if (lnf) hipLaunchKernelGGL((gemm_splitk<T, NWS, false, true, TO>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((gemm_splitk<T, NWS, false, false, TO>), grid, block, 0, stream, a);
  }
  return static_cast<int>(hipGetLastError());
}

#ifndef MI355_GEMM_PERSIST
#define MI355_GEMM_PERSIST 1
#endif

// compute units of the current device (persistent grids), looked up once per device
int cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64 && cache[dev] > 0) return cache[dev];
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev < 64) cache[dev] = n;
  return n;
}

template <typename T, typename TO, int BM, int BN, int WM, int WN, bool INT8>
int launch_gemm(const GemmArgs& a, hipStream_t stream) {
  if constexpr (!INT8 && sizeof(T) == 2) {
    // small 16-bit problems: the split-K kernel (see gemm_splitk)
    if (((a.M + 31) / 32) * ((a.N + 31) / 32) <= 512) {
      if (a.kb_out) return MI355_E_UNSUPPORTED;  // no key-bound epilogue there
      return launch_gemm_splitk<T, TO>(a, stream);
    }
  }
  // the key-bound epilogue: 16-bit outputs of the 256 x 256 tiles
  if (a.kb_out && (INT8 || sizeof(T) != 2 || sizeof(TO) != 2 || BM != 256 || BN != 256))
    return MI355_E_UNSUPPORTED;
  const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  if (tiles <= 0) return MI355_OK;
  if (tiles > 0x7fffffffLL) return MI355_E_BAD_SIZE;
  constexpr int64_t BK = MI355_GEMM_CHD * Mfma<T>::ELEMS_PER_CHUNK;  // K step of the direct path
  const dim3 grid(static_cast<unsigned>(tiles)), block(WM * WN * 64);
  // direct path: K a whole number of steps, and a tile's rows (256 x pitch) addressable with
  // 32-bit buffer offsets
  const bool direct = MI355_GEMM_DIRECT && a.K % BK == 0 &&
                      a.lda * static_cast<int64_t>(sizeof(T)) <= (int64_t{1} << 23) &&
                      a.ldw * static_cast<int64_t>(sizeof(T)) <= (int64_t{1} << 23);
  // GELU is a compile-time variant (as a run-time option its inlined code in the unrolled
  // epilogue slowed every projection by ~10%)
  const bool gelu = (a.epi & EPI_GELU) != 0;
  if constexpr (!INT8) {
    // persistent tiles (see gemm_kernel) for short K (at most 512: 8 K steps, where the per-tile
    // prologue and epilogue are a third of a tile's time) and more than two tiles per CU; K a
    // whole number of ring turns; outputs (and residual) in 16-byte aligned rows of whole 16-byte
    // groups. Measured against one tile per work-group: C5's out projection (K = N = 512) +5-8%,
    // its QKV projection +1-2%; at K = 1024 -2..+2%, at K = 2048 (C3) 6-26% slower.
    constexpr int64_t EPC_OUT = 16 / static_cast<int64_t>(sizeof(TO));
    const int ncu = MI355_GEMM_PERSIST && direct && a.K <= 512 ? cu_count() : 0;
    const bool persist = ncu > 0 && tiles > 2 * static_cast<int64_t>(ncu) && (a.K / BK) % MI355_GEMM_NST == 0 &&
                         a.N % EPC_OUT == 0 && a.ldc % EPC_OUT == 0 && aligned16(a.C) &&
                         (!a.R || (a.ldr % EPC_OUT == 0 && aligned16(a.R)));
    // (16-bit operands; the LayerNorm fold only for the output types its tiled path takes)
    constexpr bool LNF_TO = __is_same(T, TO) || __is_same(TO, _Float16);
    const bool lnf = a.ln_stats != nullptr;
    if (persist && (LNF_TO || !lnf)) {
      if (a.kb_out) return MI355_E_UNSUPPORTED;  // the persistent epilogue has no key bounds
      if constexpr (sizeof(T) == 2) {
        const dim3 pgrid(static_cast<unsigned>(ncu));
        if (lnf) {
          if constexpr (LNF_TO) {
            if (gelu)
              hipLaunchKernelGGL((gemm_kernel<T, TO, BM, BN, WM, WN, false, true, true, true, true>), pgrid, block, 0, stream, a);
            else
              hipLaunchKernelGGL((gemm_kernel<T, TO, BM, BN, WM, WN, false, true, false, true, true>), pgrid, block, 0, stream, a);
          }
        } else if (gelu)
          hipLaunchKernelGGL((gemm_kernel<T, TO, BM, BN, WM, WN, false, true, true, false, true>), pgrid, block, 0, stream, a);
        else
          hipLaunchKernelGGL((gemm_kernel<T, TO, BM, BN, WM, WN, false, true, false, false, true>), pgrid, block, 0, stream, a);
        return static_cast<int>(hipGetLastError());
      }
    }
    // the LayerNorm fold, likewise a compile-time variant (16-bit QKV / FFN-in outputs keep
    // their input type or the fp16 attention core type; fp32 stays fp32)
    constexpr bool LNF_OK = __is_same(T, TO) || __is_same(TO, _Float16);
    if (a.ln_stats != nullptr) {
      if constexpr (LNF_OK) {
        if (direct && gelu)
          hipLaunchKernelGGL((gemm_kernel<T, TO, BM, BN, WM, WN, false, true, true, true>), grid, block, 0, stream, a);
        else if (direct)
          hipLaunchKernelGGL((gemm_kernel<T, TO, BM, BN, WM, WN, false, true, false, true>), grid, block, 0, stream, a);
        else if (gelu)
          hipLaunchKernelGGL((gemm_kernel<T, TO, BM, BN, WM, WN, false, false, true, true>), grid, block, 0, stream, a);
        else
          hipLaunchKernelGGL((gemm_kernel<T, TO, BM, BN, WM, WN, false, false, false, true>), grid, block, 0, stream, a);
        return static_cast<int>(hipGetLastError());
      } else {
        return MI355_E_UNSUPPORTED;
      }
    }
  }
  if (direct && gelu)
    hipLaunchKernelGGL((gemm_kernel<T, TO, BM, BN, WM, WN, INT8, true, true, false>), grid, block, 0, stream, a);
  else if (direct)
    hipLaunchKernelGGL((gemm_kernel<T, TO, BM, BN, WM, WN, INT8, true, false, false>), grid, block, 0, stream, a);
  else if (gelu)
    hipLaunchKernelGGL((gemm_kernel<T, TO, BM, BN, WM, WN, INT8, false, true, false>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((gemm_kernel<T, TO, BM, BN, WM, WN, INT8, false, false, false>), grid, block, 0, stream, a);
  return static_cast<int>(hipGetLastError());
}

}  // namespace

// 16-bit / int8 work-group tile 256 x 256; wave grid overridable at build time
#ifndef MI355_GEMM_BM
#define MI355_GEMM_BM 256
#endif
#ifndef MI355_GEMM_BN
#define MI355_GEMM_BN 256
#endif
#ifndef MI355_GEMM_WM
#define MI355_GEMM_WM 4
#endif
#ifndef MI355_GEMM_WN
#define MI355_GEMM_WN 2
#endif

template <typename T, int BM, int BN, int WM, int WN, bool INT8>
int launch_by_out(const GemmArgs& a, hipStream_t s) {
  switch (a.out_dtype) {
    case MI355_F16: return launch_gemm<T, _Float16, BM, BN, WM, WN, INT8>(a, s);
    case MI355_BF16: return launch_gemm<T, __bf16, BM, BN, WM, WN, INT8>(a, s);
    default: return launch_gemm<T, float, BM, BN, WM, WN, INT8>(a, s);
  }
}

namespace {
int gemm_bias_impl(int in_dtype, int out_dtype, const void* A, int64_t lda, const void* W, int64_t ldw,
                   const float* bias, const void* R, int64_t ldr, void* C, int64_t ldc, int64_t M,
                   int64_t N, int64_t K, const uint8_t* row_valid, void* stream, int epi = 0,
                   const float* ln_stats = nullptr, const float* ln_colsum = nullptr,
                   const GemmArgs* kb = nullptr) {
  if (M < 0 || N < 0 || K < 0) return MI355_E_BAD_SIZE;
  if (M == 0 || N == 0) return MI355_OK;
  if (!A || !W || !C) return MI355_E_NULL_POINTER;
  const bool ok_in = in_dtype == MI355_F32 || in_dtype == MI355_F16 || in_dtype == MI355_BF16;
  const bool ok_out = out_dtype == MI355_F32 || out_dtype == MI355_F16 || out_dtype == MI355_BF16;
  if (!ok_in || !ok_out) return MI355_E_BAD_DTYPE;
  // fp32 inputs give fp32 or fp16 (the attention core type of an fp32 model's fp16 core);
  // 16-bit inputs give either 16-bit type or fp32
  if (in_dtype == MI355_F32 && out_dtype == MI355_BF16) return MI355_E_UNSUPPORTED;
  const int64_t epc = in_dtype == MI355_F32 ? 4 : 8;
  if (K % epc || lda % epc || ldw % epc || !aligned16(A) || !aligned16(W))
    return MI355_E_ALIGNMENT;
  if (lda < K || ldw < K || ldc < N || (R && ldr < N)) return MI355_E_BAD_SIZE;
  GemmArgs a{};
  a.A = A;
  a.W = W;
  a.bias = bias;
  a.C = C;
  a.R = R;
  a.row_valid = row_valid;
  a.lda = lda;
  a.ldw = ldw;
  a.ldc = ldc;
  a.ldr = ldr;
  a.M = M;
  a.N = N;
  a.K = K;
  a.out_dtype = out_dtype;
  a.epi = epi;
  a.ln_stats = ln_stats;
  a.ln_colsum = ln_colsum;
  if (kb) {
    a.kb_out = kb->kb_out;
    a.kb_valid = kb->kb_valid;
    a.kb_col0 = kb->kb_col0;
    a.kb_seq = kb->kb_seq;
    a.kb_hd = kb->kb_hd;
    a.kb_heads = kb->kb_heads;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a.kb_out && in_dtype == MI355_F32) return MI355_E_UNSUPPORTED;
  // 16-bit tile: 256 x 256 on 8 waves, or 128 x 128 / 64 x 64 on 4 waves (two or more
  // work-groups per CU) where 256 x 256 tiles would leave CUs idle (fewer tiles than CUs:
  // MI355_GEMM_FILL) or compute half padding (at most 128 output features, the official shapes'
  // d_model 128, short of the persistent regime's tile counts, where 256 x 256 stays faster);
  // 64 x 64 where even 128 x 128 tiles would not give half the CUs one (MI355_GEMM_FILL64).
  // Measured against 256 x 256 (one process, one box): 65536 x 128 x 128 44 -> 20 us,
  // 8192 x 128 x 128 38 -> 11 us (64 x 64), 8192 x 384 x 128 19 -> 15 us, 8192 x 1024 x 1024
  // 39 -> 31 us; 1280000 x 128 x 128 (persistent) 194 us against 224 us at 128 x 128.
  int tile = 256;
  if (MI355_GEMM_NARROW && !a.kb_out) {
    const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
    const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
    if (t256 < MI355_GEMM_FILL || (N <= 128 && t256 < 4 * MI355_GEMM_FILL)) tile = 128;
    if (tile == 128 && t128 < MI355_GEMM_FILL64) tile = 64;
  }
  switch (in_dtype) {
    case MI355_F16:
      if (tile == 64) return launch_by_out<_Float16, 64, 64, 2, 2, false>(a, s);
      if (tile == 128) return launch_by_out<_Float16, 128, 128, 2, 2, false>(a, s);
      return launch_by_out<_Float16, MI355_GEMM_BM, MI355_GEMM_BN, MI355_GEMM_WM, MI355_GEMM_WN, false>(a, s);
    case MI355_BF16:
      if (tile == 64) return launch_by_out<__bf16, 64, 64, 2, 2, false>(a, s);
      if (tile == 128) return launch_by_out<__bf16, 128, 128, 2, 2, false>(a, s);
      return launch_by_out<__bf16, MI355_GEMM_BM, MI355_GEMM_BN, MI355_GEMM_WM, MI355_GEMM_WN, false>(a, s);
    default: {
      // small problems (the fp32 configuration's projections are 128 x 768 and 128 x 256):
      // 32 x 32 tiles with K split over 8 waves; mid-size ones 64 x 64 tiles
      const int64_t tiles32 = ((a.M + 31) / 32) * ((a.N + 31) / 32);
      const int64_t tiles128 = ((a.M + 127) / 128) * ((a.N + 127) / 128);
      if (out_dtype == MI355_F16) {
        if (tiles32 <= 512) return launch_gemm_splitk<float, _Float16>(a, s);
        if (tiles128 < MI355_GEMM_F32_FILL) return launch_gemm<float, _Float16, 64, 64, 2, 2, false>(a, s);
        return launch_gemm<float, _Float16, 128, 128, 2, 2, false>(a, s);
      }
      if (tiles32 <= 512) return launch_gemm_splitk<float, float>(a, s);
      if (tiles128 < MI355_GEMM_F32_FILL) return launch_gemm<float, float, 64, 64, 2, 2, false>(a, s);
      return launch_gemm<float, float, 128, 128, 2, 2, false>(a, s);
    }
  }
}
}  // namespace

extern "C" int mi355_gemm_bias(int in_dtype, int out_dtype, const void* A, int64_t lda,
                               const void* W, int64_t ldw, const float* bias, void* C, int64_t ldc,
                               int64_t M, int64_t N, int64_t K, const uint8_t* row_valid,
                               void* stream) {
  return gemm_bias_impl(in_dtype, out_dtype, A, lda, W, ldw, bias, nullptr, 0, C, ldc, M, N, K,
                        row_valid, stream);
}

extern "C" int mi355_gemm_bias_residual(int in_dtype, int out_dtype, const void* A, int64_t lda,
                                        const void* W, int64_t ldw, const float* bias, const void* R,
                                        int64_t ldr, void* C, int64_t ldc, int64_t M, int64_t N,
                                        int64_t K, const uint8_t* row_valid, void* stream) {
  if (M > 0 && N > 0 && !R) return MI355_E_NULL_POINTER;
  return gemm_bias_impl(in_dtype, out_dtype, A, lda, W, ldw, bias, R, ldr, C, ldc, M, N, K,
                        row_valid, stream);
}

extern "C" int mi355_gemm_bias_gelu(int in_dtype, int out_dtype, const void* A, int64_t lda,
                                    const void* W, int64_t ldw, const float* bias, void* C,
                                    int64_t ldc, int64_t M, int64_t N, int64_t K, void* stream) {
  return gemm_bias_impl(in_dtype, out_dtype, A, lda, W, ldw, bias, nullptr, 0, C, ldc, M, N, K,
                        nullptr, stream, EPI_GELU);
}

extern "C" int mi355_gemm_bias_residual_zero_masked(int in_dtype, int out_dtype, const void* A,
                                                    int64_t lda, const void* W, int64_t ldw,
                                                    const float* bias, const void* R, int64_t ldr,
                                                    void* C, int64_t ldc, int64_t M, int64_t N,
                                                    int64_t K, const uint8_t* row_valid,
                                                    void* stream) {
  if (M > 0 && N > 0 && !R) return MI355_E_NULL_POINTER;
  return gemm_bias_impl(in_dtype, out_dtype, A, lda, W, ldw, bias, R, ldr, C, ldc, M, N, K,
                        row_valid, stream, EPI_ZERO_MASKED);
}

namespace {
// Checks of the key-bound arguments (mi355_*_kbound); fills kb's key-bound fields. The epilogue
// writes whole 256-key chunks with plain stores, so a chunk must be one tile's rows (seq_len a
// multiple of 256) and a tile's columns whole heads of the K block (k_col0 and n_heads *
// head_dim multiples of 256); its 16-byte copy path needs 16-byte aligned output rows.
int kb_args(GemmArgs& kb, int out_dtype, const void* C, int64_t ldc, int64_t M, int64_t N,
            float* key_bounds, int64_t k_col0, int64_t n_heads, int64_t head_dim, int64_t seq_len,
            const uint8_t* key_valid) {
  if (!key_bounds) return MI355_E_NULL_POINTER;
  if (reinterpret_cast<uintptr_t>(key_bounds) & 3u) return MI355_E_ALIGNMENT;
  if (n_heads <= 0 || seq_len <= 0 || k_col0 < 0 || n_heads > (1 << 20)) return MI355_E_BAD_SIZE;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128) return MI355_E_HEAD_DIM;
  if (k_col0 + n_heads * head_dim > N || M % seq_len != 0) return MI355_E_BAD_SIZE;
  if (out_dtype != MI355_F16 && out_dtype != MI355_BF16) return MI355_E_UNSUPPORTED;
  if (seq_len % 256 != 0 || k_col0 % 256 != 0 || (n_heads * head_dim) % 256 != 0)
    return MI355_E_UNSUPPORTED;
  if (ldc % 8 != 0 || !aligned16(C)) return MI355_E_UNSUPPORTED;
  kb.kb_out = key_bounds;
  kb.kb_valid = key_valid;
  kb.kb_col0 = k_col0;
  kb.kb_seq = seq_len;
  kb.kb_hd = static_cast<int>(head_dim);
  kb.kb_heads = static_cast<int>(n_heads);
  return MI355_OK;
}
}  // namespace

extern "C" int mi355_gemm_bias_kbound(int in_dtype, int out_dtype, const void* A, int64_t lda,
                                      const void* W, int64_t ldw, const float* bias, void* C,
                                      int64_t ldc, int64_t M, int64_t N, int64_t K,
                                      float* key_bounds, int64_t k_col0, int64_t n_heads,
                                      int64_t head_dim, int64_t seq_len,
                                      const uint8_t* key_valid, void* stream) {
  if (M < 0 || N < 0 || K < 0) return MI355_E_BAD_SIZE;
  if (M == 0 || N == 0) return MI355_OK;
  GemmArgs kb{};
  const int rc = kb_args(kb, out_dtype, C, ldc, M, N, key_bounds, k_col0, n_heads, head_dim,
                         seq_len, key_valid);
  if (rc != MI355_OK) return rc;
  return gemm_bias_impl(in_dtype, out_dtype, A, lda, W, ldw, bias, nullptr, 0, C, ldc, M, N, K,
                        nullptr, stream, 0, nullptr, nullptr, &kb);
}

namespace {
// Checks shared by the LayerNorm-folded entry points; 0 when the arguments are acceptable.
int ln_gemm_check(int in_dtype, int out_dtype, const void* X, int64_t ldx, const void* W,
                  const float* colsum, float eps, void* C, int64_t M, int64_t N, int64_t K, int epi) {
  if (M < 0 || N < 0 || K <= 0) return MI355_E_BAD_SIZE;
  if (M == 0 || N == 0) return MI355_OK;
  if (!X || !W || !C || !colsum) return MI355_E_NULL_POINTER;
  if (in_dtype != MI355_F32 && in_dtype != MI355_F16 && in_dtype != MI355_BF16) return MI355_E_BAD_DTYPE;
  if (out_dtype != MI355_F32 && out_dtype != MI355_F16 && out_dtype != MI355_BF16) return MI355_E_BAD_DTYPE;
  // 16-bit outputs: the input type, or fp16 (the attention core type of a bf16 model)
  if (in_dtype != out_dtype && out_dtype != MI355_F16) return MI355_E_UNSUPPORTED;
  if (epi & ~MI355_EPI_GELU) return MI355_E_UNSUPPORTED;
  if (!(eps >= 0.f)) return MI355_E_BAD_SIZE;
  const int64_t epv = in_dtype == MI355_F32 ? 4 : 8;
  if (K % epv || ldx % epv || !aligned16(X)) return MI355_E_ALIGNMENT;
  if (ldx < K) return MI355_E_BAD_SIZE;
  if (K / epv > 64 * 16) return MI355_E_UNSUPPORTED;  // the statistics pass holds a row per wave
  return MI355_OK;
}

int ln_gemm_run(int in_dtype, int out_dtype, const void* X, int64_t ldx, const void* W, int64_t ldw,
                const float* colsum, const float* bias, float eps, float* stats, void* C,
                int64_t ldc, int64_t M, int64_t N, int64_t K, int epi, void* stream,
                const GemmArgs* kb = nullptr) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = mi355_internal_ln_stats(in_dtype, X, ldx, eps, stats, M, K, s);
  if (rc != MI355_OK) return rc;
  return gemm_bias_impl(in_dtype, out_dtype, X, ldx, W, ldw, bias, nullptr, 0, C, ldc, M, N, K,
                        nullptr, stream, (epi & MI355_EPI_GELU) ? EPI_GELU : 0, stats, colsum,
                        kb);
}
}  // namespace

extern "C" int mi355_layernorm_gemm_bias(int in_dtype, int out_dtype, const void* X, int64_t ldx,
                                         const void* W, int64_t ldw, const float* colsum,
                                         const float* bias, float eps, float* stats, void* C,
                                         int64_t ldc, int64_t M, int64_t N, int64_t K, int epi,
                                         void* stream) {
  int rc = ln_gemm_check(in_dtype, out_dtype, X, ldx, W, colsum, eps, C, M, N, K, epi);
  if (rc != MI355_OK || M == 0 || N == 0) return rc;
  if (!stats) return MI355_E_NULL_POINTER;
  if (reinterpret_cast<uintptr_t>(stats) & 7u) return MI355_E_ALIGNMENT;
  return ln_gemm_run(in_dtype, out_dtype, X, ldx, W, ldw, colsum, bias, eps, stats, C, ldc, M, N,
                     K, epi, stream);
}

extern "C" int mi355_layernorm_gemm_bias_kbound(int in_dtype, int out_dtype, const void* X,
                                                int64_t ldx, const void* W, int64_t ldw,
                                                const float* colsum, const float* bias, float eps,
                                                float* stats, void* C, int64_t ldc, int64_t M,
                                                int64_t N, int64_t K, float* key_bounds,
                                                int64_t k_col0, int64_t n_heads, int64_t head_dim,
                                                int64_t seq_len, const uint8_t* key_valid,
                                                void* stream) {
  int rc = ln_gemm_check(in_dtype, out_dtype, X, ldx, W, colsum, eps, C, M, N, K, 0);
  if (rc != MI355_OK || M == 0 || N == 0) return rc;
  if (!stats) return MI355_E_NULL_POINTER;
  if (reinterpret_cast<uintptr_t>(stats) & 7u) return MI355_E_ALIGNMENT;
  GemmArgs kb{};
  rc = kb_args(kb, out_dtype, C, ldc, M, N, key_bounds, k_col0, n_heads, head_dim, seq_len,
               key_valid);
  if (rc != MI355_OK) return rc;
  // the key-bound epilogue runs on 16-bit operands only: refuse before the statistics pass
  if (in_dtype == MI355_F32) return MI355_E_UNSUPPORTED;
  return ln_gemm_run(in_dtype, out_dtype, X, ldx, W, ldw, colsum, bias, eps, stats, C, ldc, M, N,
                     K, 0, stream, &kb);
}

// ---- the allocation-free variant: row statistics in a file-scope device array
// Each GPU the library runs on holds its own copy of `scratch` (MI355_NOALLOC_MAX_ROWS rows of
// (mean, rstd): 8 MiB) until the process ends. Host code never passes the array's name to a
// kernel (on the host it is only a stand-in for the symbol): it uses the device address that
// hipGetSymbolAddress returns for the current device, looked up once per device.
static __device__ __align__(256) float scratch[2 * MI355_NOALLOC_MAX_ROWS];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// device address of `scratch` on the device that owns `stream` (the current device for the
// null stream); nullptr after a HIP error, whose code goes to *rc
float* scratch_for(hipStream_t stream, int* rc) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) { *rc = static_cast<int>(e); return nullptr; }
  int dev = cur;
  if (stream != nullptr) {
    e = hipStreamGetDevice(stream, &dev);
    if (e != hipSuccess) { *rc = static_cast<int>(e); return nullptr; }
  }
  if (dev < 0 || dev >= kMaxDevices) { *rc = MI355_E_UNSUPPORTED; return nullptr; }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) { *rc = static_cast<int>(e); return nullptr; }
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t e2 = hipSetDevice(cur);
      if (e == hipSuccess) e = e2;
    }
    if (e != hipSuccess || ptr == nullptr) {
      *rc = e != hipSuccess ? static_cast<int>(e) : MI355_E_NULL_POINTER;
      return nullptr;
    }
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" int mi355_layernorm_gemm_bias_noalloc(int in_dtype, int out_dtype, const void* X,
                                                 int64_t ldx, const void* W, int64_t ldw,
                                                 const float* colsum, const float* bias, float eps,
                                                 void* C, int64_t ldc, int64_t M, int64_t N,
                                                 int64_t K, int epi, void* stream) {
  int rc = ln_gemm_check(in_dtype, out_dtype, X, ldx, W, colsum, eps, C, M, N, K, epi);
  if (rc != MI355_OK || M == 0 || N == 0) return rc;
  if (M > MI355_NOALLOC_MAX_ROWS) return MI355_E_BAD_SIZE;
  float* stats = scratch_for(static_cast<hipStream_t>(stream), &rc);
  if (stats == nullptr) return rc;
  // every row's statistics are written by the statistics pass before the projection reads
  // them, so nothing left by an earlier call needs clearing
  return ln_gemm_run(in_dtype, out_dtype, X, ldx, W, ldw, colsum, bias, eps, stats, C, ldc, M, N,
                     K, epi, stream);
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
  return launch_by_out<int8_t, MI355_GEMM_BM, MI355_GEMM_BN, MI355_GEMM_WM, MI355_GEMM_WN, true>(a, static_cast<hipStream_t>(stream));
}

extern "C" int mi355_gemm_i8_epilogue(const int8_t* A, const int8_t* W, const float* s_a,
                                      const float* s_w, const float* bias, int out_dtype, void* C,
                                      int64_t ldc, const void* R, int64_t ldr, int64_t M,
                                      int64_t N, int64_t K, const uint8_t* row_valid, int epi,
                                      void* stream) {
  if (M < 0 || N < 0 || K < 0) return MI355_E_BAD_SIZE;
  if (M == 0 || N == 0) return MI355_OK;
  if (!A || !W || !C || !s_a || !s_w) return MI355_E_NULL_POINTER;
  if (out_dtype != MI355_F32 && out_dtype != MI355_F16 && out_dtype != MI355_BF16)
    return MI355_E_BAD_DTYPE;
  if (epi & ~(MI355_EPI_GELU | MI355_EPI_ZERO_MASKED)) return MI355_E_UNSUPPORTED;
  // GELU feeds an FFN's hidden layer; a residual follows only an output projection
  if ((epi & MI355_EPI_GELU) && R) return MI355_E_UNSUPPORTED;
  if (K % 16 || !aligned16(A) || !aligned16(W)) return MI355_E_ALIGNMENT;
  if (ldc < N || (R && ldr < N)) return MI355_E_BAD_SIZE;
  GemmArgs a{};
  a.A = A;
  a.W = W;
  a.bias = bias;
  a.C = C;
  a.R = R;
  a.s_a = s_a;
  a.s_w = s_w;
  a.row_valid = row_valid;
  a.lda = K;
  a.ldw = K;
  a.ldc = ldc;
  a.ldr = ldr;
  a.M = M;
  a.N = N;
  a.K = K;
  a.out_dtype = out_dtype;
  a.epi = (epi & MI355_EPI_GELU ? EPI_GELU : 0) | (epi & MI355_EPI_ZERO_MASKED ? EPI_ZERO_MASKED : 0);
  return launch_by_out<int8_t, MI355_GEMM_BM, MI355_GEMM_BN, MI355_GEMM_WM, MI355_GEMM_WN, true>(a, static_cast<hipStream_t>(stream));
}
