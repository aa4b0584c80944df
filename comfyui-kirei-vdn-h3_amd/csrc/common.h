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

// Round to nearest even (v_cvt_pk_bf16_f32 in the default rounding mode); NaN stays a NaN.
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// bf16 rounding of an fp32 value, returned as fp32.
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

// two values rounded to bf16 by one packed conversion; `lo` in the low half
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

// ---- exact SiLU in bf16 and the W8A8 quantisation codes (device) ---------------------
__device__ __forceinline__ float silu_f(float x) { return x / (1.f + expf(-x)); }

// True when fp32 value y lies within 32 ulp of a bf16 rounding midpoint (its low 16 bits
// near 0x8000): only there can an approximation with a smaller error round differently.
__device__ __forceinline__ bool near_bf16_midpoint(float y) {
  return ((__float_as_uint(y) & 0xffffu) - 0x7fe0u) < 0x40u;
}

// bf16(SiLU(x)) as fp32, bit-identical to round_bf(silu_f(x)): the hardware exp2 / reciprocal
// form is within ~15 ulp of x / (1 + e^-x) for |x| <= 16 (argument rounding of -x log2(e),
// v_exp_f32, 1 + e, v_rcp_f32, the product), so it rounds to the same bf16 value unless it
// lies near a midpoint; those values and |x| > 16 take the exact expression.
__device__ __forceinline__ float silu_bf(float x) {
  const float y = x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
  if (__builtin_expect(fabsf(x) > 16.f || near_bf16_midpoint(y), 0)) return round_bf(silu_f(x));
  return round_bf(y);
}

constexpr float kF8Max = 448.f;
constexpr float kI8Max = 127.f;

// fp32 (finite, |x| <= 448) -> OCP e4m3fn code, round to nearest even.
__device__ __forceinline__ uint32_t e4m3_code(float x) {
  const uint32_t sign = (__float_as_uint(x) >> 24) & 0x80u;
  const float a = fabsf(x);
  uint32_t code;
  if (a < 0.015625f) {
    // zero and subnormals: multiples of 2^-9; rounding up to 8 gives the smallest normal (0x08)
    code = (uint32_t)rintf(a * 512.f);
  } else {
    uint32_t ua = __float_as_uint(a);
    ua += 0x7ffffu + ((ua >> 20) & 1u);  // keep 3 mantissa bits, ties to even (carries into the exponent)
    code = (((ua >> 23) - 120u) << 3) | ((ua >> 20) & 7u);
  }
  return sign | code;
}

// int8 code of x / scale: round half to even, clamp to +-127
__device__ __forceinline__ uint32_t i8_code(float x) {
  return (uint32_t)(int32_t)fminf(fmaxf(rintf(x), -kI8Max), kI8Max) & 0xffu;
}

// x / s for the activation quantisations, where s = max(amax / qmax, 1e-12), amax is the largest |x|
// of the bf16 values being quantised and r = 1 / s (correctly rounded): x * r with one FMA
// correction, the sign of x kept. For every finite bf16 amax and every bf16 x with |x| <= amax
// (1.07e9 pairs for each of qmax = 127 and 448) the int8 and e4m3 codes of this quotient equal those
// of the correctly rounded x / s, checked exhaustively (tests/quant_division_check.c); the quotient
// itself may differ in its last bit. Four instructions instead of a division's ten or so. Callers
// keep the division for a non-finite amax, where x * r would give NaN instead of the division's 0.
__device__ __forceinline__ float quant_div(float x, float s, float r) {
  const float q0 = x * r;
  return copysignf(fmaf(fmaf(-s, q0, x), r, q0), x);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// ---- MFMA wrappers ------------------------------------------------------------------
// 32x32x16 bf16 -> fp32. Lane l holds A[m = l%32][k = 8*(l/32) + j], B[k = 8*(l/32) + j][n = l%32]
// for j = 0..7, and C[m = 8*(i/4) + 4*(l/32) + i%4][n = l%32] for i = 0..15.
__device__ __forceinline__ f32x16_t mfma_bf16_32x32x16(bf16x8_t a, bf16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// 16x16x32 bf16 -> fp32. Lane l holds A[m = l%16][k = 8*(l/16) + j], B[k = 8*(l/16) + j][n = l%16]
// for j = 0..7, and C[m = 4*(l/16) + i][n = l%16] for i = 0..3.
__device__ __forceinline__ f32x4_t mfma_bf16_16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// 16-byte vector load / store (addresses must be 16-byte aligned).
__device__ __forceinline__ u32x4_t ld16(const void *p) { return *reinterpret_cast<const u32x4_t *>(p); }
__device__ __forceinline__ void st16(void *p, u32x4_t v) { *reinterpret_cast<u32x4_t *>(p) = v; }
// the same to global memory with the non-temporal hint: the data streams through L2 without
// displacing lines that other workgroups are still reading
__device__ __forceinline__ void st16_stream(void *p, u32x4_t v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t *>(p));
}
// 16-byte global load with the non-temporal hint, for data read once
__device__ __forceinline__ u32x4_t ld16_stream(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
}

// ---- direct-to-LDS tile loads and explicit waits ---------------------------------------
// s_waitcnt with vmcnt <= N, lgkmcnt = 0 (expcnt left alone), gfx9 encoding of the immediate.
template <int N>
__device__ __forceinline__ void wait_vm_lds() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | ((N >> 4) << 14));
}

// Workgroup barrier without the fence of __syncthreads (which would also wait for every
// in-flight tile load); the empty asm statements keep the compiler from moving memory
// accesses across it. The waits the step needs are issued explicitly before it.
__device__ __forceinline__ void bare_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// 16 bytes per lane from global memory straight into LDS (global_load_lds_dwordx4): lane i of the
// wave writes lds_wave_base + 16 i; lds_wave_base must be the same for the whole wave. Issued
// as inline assembly so that the compiler does not add its own conservative "wait for every
// LDS DMA" before each LDS read: the kernel orders these loads itself, with explicit vmcnt
// waits and barriers. M0 is a reserved register the compiler does not preserve around the
// statement; no kernel of this library uses M0 otherwise (the generated code has no other M0
// access).
__device__ __forceinline__ uint32_t lds_address(const void *p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void *)(p)));
}
// the same with the wave's LDS byte address given directly (wave-uniform)
__device__ __forceinline__ void global_to_lds16_at(const void *src, uint32_t lds_wave_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src),
               "s"(__builtin_amdgcn_readfirstlane(lds_wave_addr))
               : "m0");
}
__device__ __forceinline__ void global_to_lds16(const void *src, void *lds_wave_base) {
  global_to_lds16_at(src, lds_address(lds_wave_base));
}
// the same with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane byte offset
// (the scalar-base form of the instruction: no 64-bit per-lane address). `sbase` must be the
// same for the whole wave; it is read from the first active lane.
__device__ __forceinline__ void global_to_lds16_sbase(const void *sbase, uint32_t lane_bytes,
                                                      uint32_t lds_wave_addr) {
  const uint64_t b = reinterpret_cast<uintptr_t>(sbase);
  // the builtin returns a signed int: go through uint32_t so the low half is zero-extended
  const uint64_t ub = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b) |
                      ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(lane_bytes), "s"(ub),
               "s"(__builtin_amdgcn_readfirstlane(lds_wave_addr))
               : "m0");
}

}  // namespace vdnh3

#define VDNH3_HOST_CHECK(expr, code, ...)                 \
  do {                                                    \
    if (!(expr)) return ::vdnh3::set_error(code, __VA_ARGS__); \
  } while (0)
