// Device-side building blocks shared by the attention and delta kernels
// (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace da {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Element traits: the 32x32x16 MFMA and the fp32 <-> element conversions.
// Operands travel as raw 32-bit words so one code path serves bf16 and fp16.
template <typename T> struct Elt;

template <> struct Elt<__bf16> {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even pack of two floats (lo in bits 0..15).
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    bf16x2 v = __builtin_convertvector((f32x2){lo, hi}, bf16x2);
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  // acc + lo(w) + hi(w) in one v_dot2 (products with 1.0 are exact)
  static __device__ __forceinline__ float add_pair(uint32_t w, float acc) {
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), one, acc, false);
  }
};

template <> struct Elt<_Float16> {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    f16x2 v = __builtin_convertvector((f32x2){lo, hi}, f16x2);
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
  static __device__ __forceinline__ float add_pair(uint32_t w, float acc) {
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), one, acc, false);
  }
};

// Separates VALU producers of MFMA operands from MFMAs written as inline asm,
// which the compiler's hazard recognizer does not see: a VALU write of a
// register needs 2 wait states before an MFMA reads it. Also a scheduling
// barrier, so the producers cannot move past it.
__device__ __forceinline__ void mfma_src_fence() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 1");
  __builtin_amdgcn_sched_barrier(0);
}

// Both halves of the wave exchange a value with the lane 32 away:
// returns {x[l], x[l ^ 32]} in some order, so a symmetric combine of the
// pair (max, +) gives the same answer on both lanes.
__device__ __forceinline__ void swap32(float x, float& a, float& b) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ float max32(float x) {
  float a, b;
  swap32(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float sum32(float x) {
  float a, b;
  swap32(x, a, b);
  return a + b;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

#define DA_LDS __attribute__((address_space(3)))

// f(std::integral_constant<int, I>) for I = B .. E-1, unrolled at compile
// time (for indices that must be template arguments, e.g. register tiles)
template <int B, int E>
struct StaticFor {
  template <typename F>
  static __device__ __forceinline__ void run(F&& f) {
    if constexpr (B < E) {
      f(std::integral_constant<int, B>{});
      StaticFor<B + 1, E>::run(f);
    }
  }
};


// Streaming (non-temporal) 16- and 8-byte global accesses for data touched
// once. Used where every store instruction writes whole contiguous lines (the
// element-wise kernels); the attention epilogues write 16-byte pieces of many
// rows per instruction and measured 9 % slower with them.
__device__ __forceinline__ u32x4 ld_nt4(const void* p) { return __builtin_nontemporal_load((const u32x4*)p); }
__device__ __forceinline__ void st_nt4(void* p, u32x4 v) { __builtin_nontemporal_store(v, (u32x4*)p); }
__device__ __forceinline__ u32x2 ld_nt2(const void* p) { return __builtin_nontemporal_load((const u32x2*)p); }
__device__ __forceinline__ void st_nt2(void* p, u32x2 v) { __builtin_nontemporal_store(v, (u32x2*)p); }
typedef short s16x4 __attribute__((ext_vector_type(4)));

// Buffer resource over `bytes` bytes from `base` (raw buffer: stride 0, word 3
// = the gfx9 data-format default). Loads at offsets >= bytes return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// 16 bytes per lane from global memory straight into LDS: lane i of the wave
// writes LDS bytes [lds + 16 i, lds + 16 i + 16). `lds` must be wave-uniform.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, DA_LDS void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, voff, 0, 0, 0);
}

// Division by a divisor fixed for a launch (d >= 1) of dividends in
// [0, 2^31), by multiply and shift: q = (mulhi(n, m) + n) >> s with
// s = ceil(log2 d) and m = floor(2^32 (2^s - d) / d) + 1 (Granlund and
// Montgomery's round-up method; mulhi(n, m) <= n keeps the sum below 2^32).
// The kernels' runtime divisors (heads per tile, row tiles, KV heads, query
// block, stride) would otherwise each cost a ~30-instruction software divide.
struct FastDiv {
  uint32_t d, m, s;
};

__host__ __device__ inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  const uint64_t m = ((1ull << 32) * ((1ull << s) - d)) / d + 1;
  return FastDiv{d, (uint32_t)m, s};
}

__host__ __device__ inline uint32_t fdiv(uint32_t n, const FastDiv& f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return (__umulhi(n, f.m) + n) >> f.s;
#else
  return (uint32_t)((((uint64_t)n * f.m) >> 32) + n) >> f.s;
#endif
}

// n mod d, given q = n / d
__host__ __device__ inline uint32_t fmodq(uint32_t n, uint32_t q, const FastDiv& f) {
  return n - q * f.d;
}

// Transposed 4 x b16 LDS read: within each 16-lane group, lane i gets element
// (i % 4) of the 8-byte blocks addressed by lanes 4r + i/4, r = 0..3.
__device__ __forceinline__ u32x2 read_tr16(const DA_LDS void* p) {
  s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((DA_LDS s16x4*)p);
  return __builtin_bit_cast(u32x2, v);
}

}  // namespace da
