// Shared helpers for the gfx950 kernels of libvdnh3.so: vector types, bf16 conversion,
// MFMA wrappers and the thread-local error channel of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/vdnh3.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

namespace vdnh3 {

// ---- error channel (host) ---------------------------------------------------------
int set_error(int code, const char *fmt, ...);
int check_launch(const char *what);

// ---- bf16 <-> fp32 (device) ---------------------------------------------------------
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// Round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

// bf16 rounding of an fp32 value, returned as fp32.
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return uint32_t(f2bf(lo)) | (uint32_t(f2bf(hi)) << 16);
}

// ---- MFMA wrappers ------------------------------------------------------------------
// 32x32x16 bf16 -> fp32. Lane l holds A[m = l%32][k = 8*(l/32) + j], B[k = 8*(l/32) + j][n = l%32]
// for j = 0..7, and C[m = 8*(i/4) + 4*(l/32) + i%4][n = l%32] for i = 0..15.
__device__ __forceinline__ f32x16_t mfma_bf16_32x32x16(bf16x8_t a, bf16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// 16-byte vector load / store (addresses must be 16-byte aligned).
__device__ __forceinline__ u32x4_t ld16(const void *p) { return *reinterpret_cast<const u32x4_t *>(p); }
__device__ __forceinline__ void st16(void *p, u32x4_t v) { *reinterpret_cast<u32x4_t *>(p) = v; }

}  // namespace vdnh3

#define VDNH3_HOST_CHECK(expr, code, ...)                 \
  do {                                                    \
    if (!(expr)) return ::vdnh3::set_error(code, __VA_ARGS__); \
  } while (0)
