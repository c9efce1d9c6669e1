// Shared device-side types and helpers for the gfx950 kernels of libmi355attn.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mi355attn.h"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define MI355_DEVINL __device__ __forceinline__
// for lambdas inside kernels: a lambda left out of line takes its by-reference register arrays
// through scratch memory
#define MI355_LAMBDA_INLINE __attribute__((always_inline))

// Per-element-type traits for the 32x32 MFMA family used by every kernel here.
//   vec8  : one 16-byte MFMA operand fragment (8 x 16-bit, 16 x int8 packed in u32x4, 4 x fp32)
//   acc   : the 32x32 accumulator fragment (16 values per lane)
//   MFMAS_PER_CHUNK: how many MFMA issues consume one 16-byte fragment per lane
template <typename T>
struct Mfma;

template <>
struct Mfma<_Float16> {
  using elem = _Float16;
  using frag = f16x8;
  using acc = f32x16;
  static constexpr int ELEMS_PER_CHUNK = 8;
  static constexpr int MFMAS_PER_CHUNK = 1;
  static MI355_DEVINL acc mma(frag a, frag b, acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<__bf16> {
  using elem = __bf16;
  using frag = bf16x8;
  using acc = f32x16;
  static constexpr int ELEMS_PER_CHUNK = 8;
  static constexpr int MFMAS_PER_CHUNK = 1;
  static MI355_DEVINL acc mma(frag a, frag b, acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<int8_t> {
  using elem = int8_t;
  using frag = i32x4;  // 16 x int8
  using acc = i32x16;
  static constexpr int ELEMS_PER_CHUNK = 16;
  static constexpr int MFMAS_PER_CHUNK = 1;
  static MI355_DEVINL acc mma(frag a, frag b, acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<float> {
  using elem = float;
  using frag = f32x4;  // 4 x fp32, consumed one element per MFMA (32x32x2)
  using acc = f32x16;
  static constexpr int ELEMS_PER_CHUNK = 4;
  static constexpr int MFMAS_PER_CHUNK = 4;
  static MI355_DEVINL acc mma_elem(float a, float b, acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  static MI355_DEVINL acc mma(frag a, frag b, acc c) {
    c = mma_elem(a[0], b[0], c);
    c = mma_elem(a[1], b[1], c);
    c = mma_elem(a[2], b[2], c);
    c = mma_elem(a[3], b[3], c);
    return c;
  }
};

// Accumulator layout of the 32x32 MFMAs (D = A·B, A rows = m, B columns = n):
// lane l, register i holds D[m][n] with n = l % 32 and m = 8*(i/4) + 4*(l/32) + (i%4).
// Operand layout: lane l supplies A[m = l%32][k-slice (l/32)] and B[k-slice (l/32)][n = l%32];
// A and B always use the same k-slice mapping, so any permutation of k inside a slice is sound.
MI355_DEVINL int mfma_row(int i, int lane) { return ((i >> 2) << 3) + ((lane >> 5) << 2) + (i & 3); }

template <typename T>
MI355_DEVINL float to_f32(T v) {
  return static_cast<float>(v);
}

template <typename T>
MI355_DEVINL T from_f32(float v) {
  return static_cast<T>(v);  // round-to-nearest-even for _Float16 / __bf16
}

// Reductions over the lane pair (l, l ^ 32) with v_permlane32_swap (gfx950). Swapping a value
// with itself leaves, in every lane, {own, partner} in the two results (which one lands where
// depends on the lane half), so max/sum of the two is the pair reduction in all 64 lanes.
MI355_DEVINL float pair_max(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// LDS DMA (global -> LDS, lane i's 16 bytes at lds_addr + 16 i; 1-byte form: lane i's byte
// zero-extended at lds_addr + 4 i), issued through inline assembly so that the compiler does not
// treat it as a pending LDS write: with the builtin it makes every later LDS wait a full
// lgkmcnt(0) while the load is in flight, and adds vmcnt waits before transpose reads. Callers
// order the data themselves (s_waitcnt vmcnt + a work-group barrier before the destination is
// read) and never read a destination while its load is in flight. lds_addr must be wave-uniform.
// An SALU write of M0 needs one wait state before a load with LDS=1 reads it (the s_nop 0 the
// compiler also emits for its own LDS-DMA loads).
MI355_DEVINL void dma_lds16(const void* gptr, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr),
               "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory", "m0");
}
MI355_DEVINL void dma_lds1(const void* gptr, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_ubyte %0, off" ::"v"(gptr),
               "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory", "m0");
}
// A wave-uniform pointer held in scalar registers (the value of the wave's first lane).
template <typename P>
MI355_DEVINL P* uniform_ptr(P* ptr) {
  const uint64_t a = reinterpret_cast<uint64_t>(ptr);
  const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a)));
  const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32)));
  return reinterpret_cast<P*>(lo | (hi << 32));
}
// Raw buffer resource (base, stride 0, `bytes` records, 32-bit data format) as four wave-uniform
// dwords: loads at or past `bytes` (voffset + soffset + instruction offset) return zeros.
MI355_DEVINL u32x4 buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const auto u = [](uint32_t v) { return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(v)); };
  return u32x4{u(static_cast<uint32_t>(a)), u(static_cast<uint32_t>(a >> 32) & 0xffffu), u(bytes),
               0x00020000u};
}
// Buffer load straight into LDS (16 bytes per lane from rsrc base + voffset + soffset, landing
// at LDS lds_addr + 16 lane), issued from inline assembly for the reason given above.
MI355_DEVINL void buffer_dma_lds16(u32x4 rsrc, uint32_t voffset, uint32_t soffset, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voffset),
               "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(soffset)),
               "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory", "m0");
}
MI355_DEVINL float pair_sum(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

MI355_DEVINL int elem_size(int dtype) { return dtype == MI355_F32 ? 4 : 2; }

// Key-norm bounds (the attention's bound pass and the QKV projection's epilogue compute them the
// same way, so both give the same bits): |k|^2 of a key is a sum over its 16-byte chunks of
// chunk_sq, a chain of packed dot products accumulated in fp32 (v_dot2_f32_f16 / _bf16, in
// element-pair order), combined by chunk_tree: the pairing of a butterfly over the LK chunks
// (offsets LK/2 .. 1), which the bound pass runs across lanes with __shfl_xor and the
// projection epilogue runs within one thread.
MI355_DEVINL float chunk_sq(f16x8 f) {
  float acc = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const f16x2 pr = {f[2 * r], f[2 * r + 1]};
    acc = __builtin_amdgcn_fdot2(pr, pr, acc, false);
  }
  return acc;
}
MI355_DEVINL float chunk_sq(bf16x8 f) {
  float acc = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const bf16x2 pr = {f[2 * r], f[2 * r + 1]};
    acc = __builtin_amdgcn_fdot2_f32_bf16(pr, pr, acc, false);
  }
  return acc;
}
// s[0] after the butterfly s[i] += s[i ^ off], off = LK/2 .. 1 (the lower index of each pair is
// kept; the upper one would hold the same value)
template <int LK>
MI355_DEVINL float chunk_tree(float (&s)[LK]) {
#pragma unroll
  for (int off = LK / 2; off >= 1; off >>= 1)
#pragma unroll
    for (int i = 0; i < off; ++i) s[i] = s[i] + s[i + off];
  return s[0];
}

// Buffer load straight into LDS (buffer_load_dwordx4 ... lds): 16 bytes per lane from
// base + soffset + voffset, landing at LDS lds_base + 16 * lane. The resource covers `bytes` bytes
// from `base` (the range check includes soffset); dwords past it read as 0. The resource is built in these device functions so its type
// never appears in host-compiled code.
template <typename P>
MI355_DEVINL uint32_t lds_addr_of(P* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) const void*)(p)));
}
MI355_DEVINL __amdgpu_buffer_rsrc_t raw_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                           0x00020000 /* raw buffer, 32-bit data format */);
}
MI355_DEVINL void buffer_load_lds16(const void* base, uint32_t bytes, void* lds_base, uint32_t voffset,
                                    uint32_t soffset = 0) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(raw_rsrc(base, bytes),
                                           (__attribute__((address_space(3))) void*)lds_base, 16, voffset,
                                           soffset, 0, 0);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Row statistics pass (csrc/layernorm.hip): stats[2 m] = mean, stats[2 m + 1] = 1 / sqrt(var + eps)
// of row m of X [M, K] (dtype MI355_F32 / F16 / BF16). Library-internal; arguments are checked by
// the exported entry point that calls it.
__attribute__((visibility("hidden"))) int mi355_internal_ln_stats(int dtype, const void* X,
                                                                  int64_t ldx, float eps,
                                                                  float* stats, int64_t M,
                                                                  int64_t K, hipStream_t s);
