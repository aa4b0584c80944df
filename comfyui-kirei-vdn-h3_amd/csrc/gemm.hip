// NT GEMM for gfx950 on bf16, int8 and fp8 (OCP e4m3fn) MFMA with a fused epilogue:
//
//   C[m][n] = epi( sum_k A[m][k] * B[n][k] )          A: [M, K] (lda), B: [N, K] (ldb), K contiguous
//   epi(acc) = act( round_opt( acc * alpha * a_scale[m] * b_scale[n] + bias[n] ) )   (+ C_old when accumulating)
//
// It stands in for every projection of the hybrid block: F.linear in bf16 (gates, beta, the
// VDN to_out_linear, vdn_h3/projection.py:259-261), the fp8 `_scaled_mm(x_q, W_q^T, s_x, s_w)`
// (vdn_h3/fp8.py:254-262) and the W8A8 int8 projection with per-token x per-channel scales
// (the ComfyUI-native qkv_proj / out_proj of vdn_h3/hybrid.py:263, :535).
//
// Tiling: a workgroup of 4 wavefronts computes a 128x128 tile of C, each wavefront a 64x64
// quadrant as 2x2 blocks of 32x32 MFMA accumulators. K advances in tiles of 128 bytes per row
// (64 bf16, 128 int8 or 128 fp8 elements); both operand tiles are staged in LDS with a
// 16-byte row pad (conflict-free 16-row reads) and the next tile is prefetched into
// registers while the current one is multiplied.
//   bf16: v_mfma_f32_32x32x16_bf16, 4 k-steps of 16 B per lane per tile
//   int8: v_mfma_i32_32x32x32_i8,   4 k-steps of 16 B per lane per tile
//   fp8 : v_mfma_scale_f32_32x32x64_f8f6f4 (unit block scales), 2 k-steps of 32 B per lane
// Every lane reads its A and B k-slices at the same byte offsets, so the products pair the
// same k whatever order the instruction assigns to the lane's bytes.
#include <type_traits>

#include "common.h"

namespace vdnh3 {
namespace {

constexpr int kGemmBM = 128, kGemmBN = 128, kGemmKB = 128;  // tile rows, cols, bytes of K per tile
constexpr int kGemmThreads = 256;
constexpr int kGemmPitch = kGemmKB + 16;  // LDS row pitch in bytes

enum GemmKind { kBF16 = 0, kI8 = 1, kF8 = 2 };
enum OutType { kOutBF16 = 0, kOutF32 = 1, kOutI32 = 2 };

struct GemmEpi {
  const float *a_scale;  // [M] or null
  const float *b_scale;  // [N] or null (a single value when b_scale_n == 1)
  int b_scale_n;
  int a_scale_n;
  float alpha;
  const void *bias;  // [N] or null
  int bias_bf16;
  int act;            // 0 none, 1 sigmoid
  int out_type;       // OutType
  int accumulate;     // C += epi(acc)
  int round_linear;   // bf16 output: round the linear result to bf16 before the activation
};

__device__ __forceinline__ float sigmoidf_(float x) { return 1.f / (1.f + __expf(-x)); }

template <int KIND>
__global__ __launch_bounds__(kGemmThreads, 2) void gemm_nt_kernel(const uint8_t *__restrict__ A, int64_t lda_b,
                                                                   const uint8_t *__restrict__ B, int64_t ldb_b,
                                                                   void *__restrict__ C, int64_t ldc, int M, int N,
                                                                   int nkt, GemmEpi epi, int tiles_n) {
  __shared__ __attribute__((aligned(16))) uint8_t As[kGemmBM * kGemmPitch];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[kGemmBN * kGemmPitch];
  const int tile = blockIdx.x;
  const int tm = tile / tiles_n, tn = tile - tm * tiles_n;
  const int m0 = tm * kGemmBM, n0 = tn * kGemmBN;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

  // 4 x 16-byte chunks of each operand tile per thread: row = c >> 3, byte column = (c & 7) * 16
  const uint8_t *a_src[4];
  const uint8_t *b_src[4];
  int lds_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = tid + kGemmThreads * i, r = c >> 3, col = (c & 7) * 16;
    a_src[i] = A + (int64_t)min(m0 + r, M - 1) * lda_b + col;
    b_src[i] = B + (int64_t)min(n0 + r, N - 1) * ldb_b + col;
    lds_off[i] = r * kGemmPitch + col;
  }
  u32x4_t areg[4], breg[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    areg[i] = ld16(a_src[i]);
    breg[i] = ld16(b_src[i]);
  }

  using acc_t = typename std::conditional<KIND == kI8, i32x16_t, f32x16_t>::type;
  acc_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = acc_t{};

  for (int kt = 0; kt < nkt; ++kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      st16(As + lds_off[i], areg[i]);
      st16(Bs + lds_off[i], breg[i]);
    }
    __syncthreads();
    if (kt + 1 < nkt) {
      const int64_t off = (int64_t)(kt + 1) * kGemmKB;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        areg[i] = ld16(a_src[i] + off);
        breg[i] = ld16(b_src[i] + off);
      }
    }
    if constexpr (KIND == kF8) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        i32x8_t av[2], bv[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const uint8_t *pa = As + (wm + 32 * i + l32) * kGemmPitch + 64 * ks + 32 * g;
          const uint8_t *pb = Bs + (wn + 32 * i + l32) * kGemmPitch + 64 * ks + 32 * g;
          u32x4_t a0 = ld16(pa), a1 = ld16(pa + 16), b0 = ld16(pb), b1 = ld16(pb + 16);
          av[i] = i32x8_t{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
          bv[i] = i32x8_t{(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av[i], bv[j], acc[i][j], 0, 0, 0, 127, 0,
                                                                        127);
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        u32x4_t av[2], bv[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          av[i] = ld16(As + (wm + 32 * i + l32) * kGemmPitch + 32 * ks + 16 * g);
          bv[i] = ld16(Bs + (wn + 32 * i + l32) * kGemmPitch + 32 * ks + 16 * g);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            if constexpr (KIND == kBF16)
              acc[i][j] = mfma_bf16_32x32x16(as_bf16x8(av[i]), as_bf16x8(bv[j]), acc[i][j]);
            else
              acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4_t, av[i]),
                                                                __builtin_bit_cast(i32x4_t, bv[j]), acc[i][j], 0, 0,
                                                                0);
          }
      }
    }
    __syncthreads();
  }

  // epilogue: lane holds C[m = 8*(r/4) + 4*g + r%4][n = l32] of each 32x32 block
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn + 32 * j + l32;
    if (n >= N) continue;
    float bs = epi.alpha;
    if (epi.b_scale) bs *= epi.b_scale[epi.b_scale_n == 1 ? 0 : n];
    float bias = 0.f;
    if (epi.bias) bias = epi.bias_bf16 ? bf2f(static_cast<const uint16_t *>(epi.bias)[n])
                                       : static_cast<const float *>(epi.bias)[n];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
        if (m >= M) continue;
        const int64_t off = (int64_t)m * ldc + n;
        if (epi.out_type == kOutI32) {
          static_cast<int32_t *>(C)[off] = (int32_t)acc[i][j][r];
          continue;
        }
        float v = (float)acc[i][j][r];
        if (epi.a_scale) v *= epi.a_scale[epi.a_scale_n == 1 ? 0 : m];
        v = v * bs + bias;
        if (epi.out_type == kOutF32) {
          if (epi.act == 1) v = sigmoidf_(v);
          float *cp = static_cast<float *>(C) + off;
          *cp = epi.accumulate ? *cp + v : v;
        } else {
          if (epi.round_linear) v = round_bf(v);
          if (epi.act == 1) v = sigmoidf_(v);
          uint16_t *cp = static_cast<uint16_t *>(C) + off;
          if (epi.accumulate) v = bf2f(*cp) + round_bf(v);
          *cp = f2bf(v);
        }
      }
  }
}

template <int KIND>
int launch_gemm(const void *A, int64_t lda, const void *B, int64_t ldb, void *C, int64_t ldc, int M, int N, int K,
                const GemmEpi &epi, hipStream_t stream) {
  const int eb = KIND == kBF16 ? 2 : 1;
  const int64_t kb = (int64_t)K * eb;
  VDNH3_HOST_CHECK(M > 0 && N > 0 && K > 0, VDNH3_ERR_INVALID, "gemm: M, N, K must be positive (%d, %d, %d)", M, N,
                   K);
  VDNH3_HOST_CHECK(kb % kGemmKB == 0, VDNH3_ERR_INVALID,
                   "gemm: K * element size must be a multiple of %d bytes (K=%d)", kGemmKB, K);
  VDNH3_HOST_CHECK((lda * eb) % 16 == 0 && (ldb * eb) % 16 == 0 && lda >= K && ldb >= K && ldc >= N,
                   VDNH3_ERR_INVALID, "gemm: leading dimensions must cover K/N and be 16-byte multiples");
  VDNH3_HOST_CHECK(reinterpret_cast<uintptr_t>(A) % 16 == 0 && reinterpret_cast<uintptr_t>(B) % 16 == 0,
                   VDNH3_ERR_INVALID, "gemm: A and B must be 16-byte aligned");
  const int tiles_m = (M + kGemmBM - 1) / kGemmBM, tiles_n = (N + kGemmBN - 1) / kGemmBN;
  hipLaunchKernelGGL(gemm_nt_kernel<KIND>, dim3(tiles_m * tiles_n), dim3(kGemmThreads), 0, stream,
                     static_cast<const uint8_t *>(A), lda * eb, static_cast<const uint8_t *>(B), ldb * eb, C, ldc, M,
                     N, int(kb / kGemmKB), epi, tiles_n);
  return check_launch("gemm_nt");
}

}  // namespace
}  // namespace vdnh3

extern "C" int vdnh3_gemm(int kind, const void *A, int64_t lda, const void *B, int64_t ldb, void *C, int64_t ldc,
                          int M, int N, int K, const float *a_scale, int a_scale_n, const float *b_scale,
                          int b_scale_n, float alpha, const void *bias, int bias_bf16, int act, int out_type,
                          int accumulate, int round_linear, void *stream) {
  using namespace vdnh3;
  VDNH3_HOST_CHECK(A && B && C, VDNH3_ERR_INVALID, "gemm: null operand");
  VDNH3_HOST_CHECK(out_type >= kOutBF16 && out_type <= kOutI32, VDNH3_ERR_INVALID, "gemm: bad out_type %d", out_type);
  VDNH3_HOST_CHECK(out_type != kOutI32 || kind == kI8, VDNH3_ERR_INVALID, "gemm: int32 output needs int8 operands");
  VDNH3_HOST_CHECK(act == 0 || act == 1, VDNH3_ERR_INVALID, "gemm: bad activation %d", act);
  VDNH3_HOST_CHECK(!a_scale || a_scale_n == 1 || a_scale_n == M, VDNH3_ERR_INVALID,
                   "gemm: a_scale must have 1 or M entries");
  VDNH3_HOST_CHECK(!b_scale || b_scale_n == 1 || b_scale_n == N, VDNH3_ERR_INVALID,
                   "gemm: b_scale must have 1 or N entries");
  GemmEpi epi{a_scale, b_scale, b_scale_n, a_scale_n, alpha, bias, bias_bf16, act, out_type, accumulate, round_linear};
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (kind) {
    case kBF16:
      return launch_gemm<kBF16>(A, lda, B, ldb, C, ldc, M, N, K, epi, s);
    case kI8:
      return launch_gemm<kI8>(A, lda, B, ldb, C, ldc, M, N, K, epi, s);
    case kF8:
      return launch_gemm<kF8>(A, lda, B, ldb, C, ldc, M, N, K, epi, s);
    default:
      return set_error(VDNH3_ERR_INVALID, "gemm: unknown operand kind %d", kind);
  }
}
