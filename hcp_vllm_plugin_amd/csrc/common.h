// Shared device helpers for the gfx950 (CDNA4) kernels of the HCP ring-attention
// hot path: element types, MFMA fragment types, 16-byte loads, conversions and
// the XCD-aware work-item remap.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hcp_mi355x.h"  // include/ is on the build's include path

namespace hcp {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kNumXcd = 8;  // MI355X: 8 XCDs, workgroups dispatched round-robin

// Element traits: 16-bit storage type, 8-wide MFMA operand type and the two
// gfx950 MFMA shapes used here (32x32x16 and 16x16x32, fp32 accumulate).
template <typename T>
struct Elem;

template <>
struct Elem<__bf16> {
  using vec8 = bf16x8;
  static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  // acc += a b with the accumulator kept in AGPRs.  The caller keeps the
  // wait states around reads and writes of acc by other instructions.
  static __device__ __forceinline__ void mfma32_acc(f32x16& acc, vec8 a, vec8 b) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  }
  static __device__ __forceinline__ uint16_t from_float(float x) {
    __bf16 h = static_cast<__bf16>(x);
    return __builtin_bit_cast(uint16_t, h);
  }
  static __device__ __forceinline__ float to_float(uint16_t x) {
    return __uint_as_float(static_cast<uint32_t>(x) << 16);
  }
};

template <>
struct Elem<_Float16> {
  using vec8 = f16x8;
  static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ void mfma32_acc(f32x16& acc, vec8 a, vec8 b) {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  }
  static __device__ __forceinline__ uint16_t from_float(float x) {
    _Float16 h = static_cast<_Float16>(x);
    return __builtin_bit_cast(uint16_t, h);
  }
  static __device__ __forceinline__ float to_float(uint16_t x) {
    return static_cast<float>(__builtin_bit_cast(_Float16, x));
  }
};

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Pack two floats into one dword of two 16-bit elements (lo = a, hi = b),
// round to nearest even: one v_cvt_pk_{bf16,f16}_f32 on gfx950.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b);
template <>
__device__ __forceinline__ uint32_t pack2<__bf16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), bf16x2));
}
template <>
__device__ __forceinline__ uint32_t pack2<_Float16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), f16x2));
}

// acc + lo + hi of a dword of two 16-bit elements, in f32: one v_dot2_f32_*
// against (1, 1), so the sum is of the rounded values themselves.
template <typename T>
__device__ __forceinline__ float sum2(uint32_t w, float acc);
template <>
__device__ __forceinline__ float sum2<__bf16>(uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w),
                                         __builtin_bit_cast(bf16x2, 0x3f803f80u), acc, false);
}
template <>
__device__ __forceinline__ float sum2<_Float16>(uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w),
                                __builtin_bit_cast(f16x2, 0x3c003c00u), acc, false);
}

// lo + hi of a dword of two 16-bit elements, in f32 (sum2 with a zero
// accumulator, as the three-operand v_dot2 with an inline 0: no register
// to clear first)
template <typename T>
__device__ __forceinline__ float sum2_first(uint32_t w);
template <>
__device__ __forceinline__ float sum2_first<__bf16>(uint32_t w) {
  float r;
  asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(r) : "v"(w), "v"(0x3f803f80u));
  return r;
}
template <>
__device__ __forceinline__ float sum2_first<_Float16>(uint32_t w) {
  float r;
  asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(w), "v"(0x3c003c00u));
  return r;
}

template <typename V>
__device__ __forceinline__ V as_vec8(u32x4 x) {
  return __builtin_bit_cast(V, x);
}

typedef const __attribute__((address_space(1))) u32x4 gu32x4;
typedef const __attribute__((address_space(1))) u32x2 gu32x2;

// Global-memory loads (global_load, not flat_load).
__device__ __forceinline__ u32x4 ldg16(const void* p) {
  return *reinterpret_cast<gu32x4*>(reinterpret_cast<uintptr_t>(p));
}
__device__ __forceinline__ u32x2 ldg8(const void* p) {
  return *reinterpret_cast<gu32x2*>(reinterpret_cast<uintptr_t>(p));
}


__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);  // v_exp_f32; exp2(-inf) = 0
}

// Reads a KV segment's token address (in elements) for token t of head h.
struct KvAddr {
  const char* k;
  const char* v;
  const int32_t* bt;
  int64_t stride_tok, stride_head, stride_block, start;
  int32_t bs_shift, bs_mask;

  __device__ __forceinline__ void init(const hcp_kv_segment& s) {
    k = reinterpret_cast<const char*>(s.k_addr);
    v = reinterpret_cast<const char*>(s.v_addr);
    bt = reinterpret_cast<const int32_t*>(s.block_table);
    stride_tok = s.stride_tok;
    stride_head = s.stride_head;
    stride_block = s.stride_block;
    start = s.start;
    int bsz = s.block_size > 0 ? s.block_size : 1;
    bs_shift = 31 - __builtin_clz(bsz);
    bs_mask = bsz - 1;
  }
  // Offset in elements of token t (segment frame) for kv head h.
  template <bool PAGED>
  __device__ __forceinline__ int64_t offset(int64_t t, int h) const {
    int64_t x = start + t;
    if constexpr (PAGED) {
      int64_t blk = bt[x >> bs_shift];
      return blk * stride_block + static_cast<int64_t>(h) * stride_head +
             (x & bs_mask) * stride_tok;
    } else {
      return x * stride_tok + static_cast<int64_t>(h) * stride_head;
    }
  }
};

// XCD-aware remap of a linear workgroup index.  Workgroups are dispatched to
// the 8 XCDs round-robin (blockIdx % 8), each XCD with its own L2.  Work items
// are (kv_head, item) with `per_kvh` items per KV head, listed heaviest
// first.  When 8 % num_kvh == 0 every XCD serves one KV head (8/num_kvh XCDs
// share a head, interleaving its items), so the K/V of a head stay in one or
// two L2s while each XCD still walks its share heaviest-first.  Returns false
// for padding workgroups.  Grid size must be xcd_grid_size(...).
__host__ __device__ inline int64_t xcd_grid_size(int64_t per_kvh, int num_kvh) {
  if (num_kvh <= kNumXcd && kNumXcd % num_kvh == 0) {
    int share = kNumXcd / num_kvh;
    int64_t per_xcd = (per_kvh + share - 1) / share;
    return per_xcd * kNumXcd;
  }
  return per_kvh * num_kvh;
}

__device__ __forceinline__ bool xcd_remap(int64_t b, int64_t per_kvh,
                                          int num_kvh, int* kvh,
                                          int64_t* item) {
  if (num_kvh <= kNumXcd && kNumXcd % num_kvh == 0) {
    int share = kNumXcd / num_kvh;
    int x = static_cast<int>(b % kNumXcd);
    int64_t s = b / kNumXcd;
    *kvh = x % num_kvh;
    int64_t i = s * share + x / num_kvh;
    *item = i;
    return i < per_kvh;
  }
  // General case: interleave heads innermost so concurrent groups share KV.
  *kvh = static_cast<int>(b % num_kvh);
  *item = b / num_kvh;
  return *item < per_kvh;
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt bits [3:0] and [15:14], expcnt
// and lgkmcnt left at "no wait")
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

}  // namespace hcp
