// clv_device.h - device-side helpers shared by the gfx950 attention kernels.
//
// Storage types are the clang builtin 16-bit floats (__bf16, _Float16) and
// float; every kernel computes in fp32. Vector types are clang ext_vector
// types so that MFMA builtins take them directly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "clv_internal.h"

namespace clv {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

__device__ __forceinline__ float fast_exp2(float x) {
  // v_exp_f32: exact 0 for -inf, 1 for 0.
  return __builtin_amdgcn_exp2f(x);
}

// ---------------------------------------------------------------- conversions
template <typename T> __device__ __forceinline__ float to_f32(T x) { return (float)x; }

template <typename T> __device__ __forceinline__ T from_f32(float x) { return (T)x; }

// Unpack a 32-bit word holding two 16-bit values (low half first).
template <typename T> __device__ __forceinline__ float lo16_to_f32(uint32_t w);
template <typename T> __device__ __forceinline__ float hi16_to_f32(uint32_t w);

template <> __device__ __forceinline__ float lo16_to_f32<__bf16>(uint32_t w) {
  return __builtin_bit_cast(float, w << 16);
}
template <> __device__ __forceinline__ float hi16_to_f32<__bf16>(uint32_t w) {
  return __builtin_bit_cast(float, w & 0xffff0000u);
}
template <> __device__ __forceinline__ float lo16_to_f32<_Float16>(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
}
template <> __device__ __forceinline__ float hi16_to_f32<_Float16>(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// ---------------------------------------------------------------- MFMA
// v_mfma_f32_16x16x32_{bf16,f16} (gfx950). Operand layout for lane l:
//   A (16 x 32, row-major M x K): row l%16, k = 8*(l/16) .. +8
//   B (32 x 16, K x N):           col l%16, k = 8*(l/16) .. +8
//   C/D (16 x 16):                col l%16, rows 4*(l/16) .. +4
template <typename T> struct Mfma16x16x32;

template <> struct Mfma16x16x32<__bf16> {
  typedef bf16x8 op_t;
  static __device__ __forceinline__ f32x4 run(op_t a, op_t b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mfma16x16x32<_Float16> {
  typedef f16x8 op_t;
  static __device__ __forceinline__ f32x4 run(op_t a, op_t b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// v_mfma_f32_16x16x16_{bf16,f16}. Operand layout for lane l:
//   A (16 x 16): row l%16, k = 4*(l/16) .. +4
//   B (16 x 16): col l%16, k = 4*(l/16) .. +4
//   C/D (16 x 16): col l%16, rows 4*(l/16) .. +4
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

template <typename T> struct Mfma16x16x16;

template <> struct Mfma16x16x16<__bf16> {
  typedef bf16x4 op_t;
  static __device__ __forceinline__ f32x4 run(op_t a, op_t b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                      __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
  }
};

template <> struct Mfma16x16x16<_Float16> {
  typedef f16x4 op_t;
  static __device__ __forceinline__ f32x4 run(op_t a, op_t b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
};

// Pack 4 fp32 values into a 4-element 16-bit MFMA operand (round to nearest even).
template <typename T>
__device__ __forceinline__ typename Mfma16x16x16<T>::op_t pack4(const float (&x)[4]) {
  typename Mfma16x16x16<T>::op_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = (T)x[i];
  return r;
}

// v_mfma_f32_32x32x16_{bf16,f16} (gfx950). Operand layout for lane l:
//   A (32 x 16): row l%32, k = 8*(l/32) .. +8
//   B (16 x 32): col l%32, k = 8*(l/32) .. +8
//   C/D (32 x 32): col l%32, rows {8*q + 4*(l/32) + r : q = 0..3, r = 0..3}
//   (register 4*q + r).
template <typename T> struct Mfma32x32x16;

template <> struct Mfma32x32x16<__bf16> {
  typedef bf16x8 op_t;
  static __device__ __forceinline__ f32x16 run(op_t a, op_t b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mfma32x32x16<_Float16> {
  typedef f16x8 op_t;
  static __device__ __forceinline__ f32x16 run(op_t a, op_t b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// Pack 8 fp32 values into an MFMA 16-bit operand (round to nearest even).
template <typename T>
__device__ __forceinline__ typename Mfma16x16x32<T>::op_t pack8(const float (&x)[8]) {
  typename Mfma16x16x32<T>::op_t r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (T)x[i];
  return r;
}

// Two 16-bit halves, one from each word: (lo(a), lo(b)) or (hi(a), hi(b)).
__device__ __forceinline__ uint32_t pair_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pair_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// ---------------------------------------------------------------- wave ops
__device__ __forceinline__ float shfl_xor(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}
__device__ __forceinline__ float shfl(float v, int src) { return __shfl(v, src, 64); }

// ---------------------------------------------------------------- memory
template <typename V>
__device__ __forceinline__ V load_vec(const void *p) {
  return *reinterpret_cast<const V *>(p);
}

template <typename V>
__device__ __forceinline__ void store_vec(void *p, V v) {
  *reinterpret_cast<V *>(p) = v;
}

// A wave-uniform 32-bit read through the scalar unit (s_load_dword). The
// compiler only emits scalar loads where it can prove no store in the kernel
// may clobber the address; kernels that store inside their main loop use this
// for read-only tables so that the read does not join the vector-memory queue
// (whose in-order counter would then also wait for every K/V load in flight).
__device__ __forceinline__ int32_t scalar_load_i32(const int32_t *ptr) {
  int32_t v;
  asm("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(ptr));
  return v;
}

// Raw buffer loads: a wave-uniform base in a buffer resource (SGPRs) plus a
// 32-bit per-lane byte offset, so the hot loops keep no 64-bit per-lane
// addresses. The range check (num_records) is set out of the way; callers
// keep every offset inside their allocation.
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void *base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7fffffff,
                                           0x00020000);
}

// A buffer resource covering [base, base + num_bytes): a raw buffer load at a
// lane offset at or past num_bytes returns zeros (the hardware range check)
// and reads no memory; num_bytes = 0 makes every lane read zeros.
__device__ __forceinline__ rsrc_t make_rsrc_range(const void *base, int num_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, num_bytes,
                                           0x00020000);
}

// Cache policy of a buffer load: kCacheDefault, or kCacheStream for data read
// exactly once (the non-temporal hint: on MI355X streaming a large buffer this
// way reads HBM at close to 90% of peak, against under 80% with the default).
constexpr int kCacheDefault = 0;
constexpr int kCacheStream = 2;

template <typename V, int AUX = kCacheDefault>
__device__ __forceinline__ V buf_load(rsrc_t r, uint32_t off);

template <> __device__ __forceinline__ u32x4 buf_load<u32x4, kCacheDefault>(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kCacheDefault));
}
template <> __device__ __forceinline__ u32x4 buf_load<u32x4, kCacheStream>(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kCacheStream));
}
template <> __device__ __forceinline__ u32x2 buf_load<u32x2, kCacheDefault>(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, kCacheDefault));
}
template <> __device__ __forceinline__ u32x2 buf_load<u32x2, kCacheStream>(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, kCacheStream));
}

}  // namespace clv
