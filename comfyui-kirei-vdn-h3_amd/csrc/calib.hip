// Sustained matrix-core throughput of the GPU on caller-supplied operand bits.
//
// The MI355X sustains its datasheet MFMA rate only while its power budget allows: the rate a
// kernel can reach depends on how many operand bits toggle. This kernel issues nothing but
// MFMAs on fragments held in registers (no memory traffic, no other VALU work in the loop), so
// its rate on random operands is the ceiling that the attention and GEMM kernels' rates can be
// read against besides the datasheet peak, and its rate on zero operands shows the clock the
// part holds when the matrix datapath barely toggles.
//
// One wavefront cycles through kFrag fragment pairs into four independent accumulators, so no
// MFMA waits for the one before it. Two workgroups of four wavefronts fill each CU.
#include "common.h"

namespace vdnh3 {
namespace {

constexpr int kCalibThreads = 256;
constexpr int kFrag = 8;  // operand fragment pairs per lane, used in turn

typedef int i32x8_v __attribute__((ext_vector_type(8)));

template <int KIND>  // 0: bf16 32x32x16, 1: int8 32x32x32, 2: fp8 e4m3 32x32x64
__global__ __launch_bounds__(kCalibThreads, 2) void mfma_peak_kernel(const i32x8_v *__restrict__ a_src,
                                                                     const i32x8_v *__restrict__ b_src, int iters,
                                                                     float *__restrict__ out) {
  const int lane = threadIdx.x & 63;
  i32x8_v a[kFrag], b[kFrag];
#pragma unroll
  for (int j = 0; j < kFrag; ++j) {
    a[j] = a_src[j * 64 + lane];
    b[j] = b_src[j * 64 + lane];
  }
  f32x16_t acc[4];
  i32x16_t iacc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    acc[j] = f32x16_t{};
    iacc[j] = i32x16_t{};
  }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < kFrag; ++j) {
      if constexpr (KIND == 0) {
        const u32x4_t av = {(uint32_t)a[j][0], (uint32_t)a[j][1], (uint32_t)a[j][2], (uint32_t)a[j][3]};
        const u32x4_t bv = {(uint32_t)b[j][0], (uint32_t)b[j][1], (uint32_t)b[j][2], (uint32_t)b[j][3]};
        acc[j & 3] = mfma_bf16_32x32x16(as_bf16x8(av), as_bf16x8(bv), acc[j & 3]);
      } else if constexpr (KIND == 1) {
        const i32x4_t av = {a[j][0], a[j][1], a[j][2], a[j][3]};
        const i32x4_t bv = {b[j][0], b[j][1], b[j][2], b[j][3]};
        iacc[j & 3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, iacc[j & 3], 0, 0, 0);
      } else {
        acc[j & 3] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[j], b[j], acc[j & 3], 0, 0, 0, 0, 0, 0);  // unscaled form, as the GEMM
      }
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) s += KIND == 1 ? (float)iacc[j][i] : acc[j][i];
  out[blockIdx.x * kCalibThreads + threadIdx.x] = s;
}

}  // namespace
}  // namespace vdnh3

extern "C" double vdnh3_mfma_peak_ops(int kind, int iters, int blocks) {
  // operations per MFMA: 2 * 32 * 32 * K with K = 16 (bf16), 32 (int8), 64 (fp8)
  const double per = kind == 0 ? 32768.0 : kind == 1 ? 65536.0 : 131072.0;
  return per * vdnh3::kFrag * (double)iters * (vdnh3::kCalibThreads / 64) * (double)blocks;
}

extern "C" int vdnh3_mfma_peak(int kind, const void *a, const void *b, int iters, int blocks, float *out,
                               void *stream) {
  VDNH3_HOST_CHECK(kind >= 0 && kind <= 2, VDNH3_ERR_INVALID, "mfma_peak: kind must be 0 (bf16), 1 (int8) or 2 (fp8)");
  VDNH3_HOST_CHECK(a != nullptr && b != nullptr && out != nullptr, VDNH3_ERR_INVALID, "mfma_peak: null pointer");
  VDNH3_HOST_CHECK(reinterpret_cast<uintptr_t>(a) % 32 == 0 && reinterpret_cast<uintptr_t>(b) % 32 == 0,
                   VDNH3_ERR_INVALID, "mfma_peak: operands must be 32-byte aligned");
  VDNH3_HOST_CHECK(iters > 0 && blocks > 0, VDNH3_ERR_INVALID, "mfma_peak: iters and blocks must be positive");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto *av = static_cast<const vdnh3::i32x8_v *>(a);
  const auto *bv = static_cast<const vdnh3::i32x8_v *>(b);
  if (kind == 0)
    hipLaunchKernelGGL(vdnh3::mfma_peak_kernel<0>, dim3(blocks), dim3(vdnh3::kCalibThreads), 0, s, av, bv, iters, out);
  else if (kind == 1)
    hipLaunchKernelGGL(vdnh3::mfma_peak_kernel<1>, dim3(blocks), dim3(vdnh3::kCalibThreads), 0, s, av, bv, iters, out);
  else
    hipLaunchKernelGGL(vdnh3::mfma_peak_kernel<2>, dim3(blocks), dim3(vdnh3::kCalibThreads), 0, s, av, bv, iters, out);
  return vdnh3::check_launch("mfma_peak");
}
