// Activation / weight quantisation passes for the W8A8 projections (HBM-bound).
//
//   rows, fp8 : scale[m] = max(amax_m / 448, 1e-12), q = e4m3fn(clamp(x / scale, +-448))
//               (vdn_h3/fp8.py:41-54 `_quantize_rows_kernel`, :99-105)
//   rows, int8: scale[m] = max(amax_m / 127, 1e-12), q = clamp(rne(x / scale), +-127)
//   tensor fp8: one scale for the whole tensor, amax by a grid reduction then a cast pass
//               (vdn_h3/fp8.py:56-71 `_absmax_kernel` + `_cast_scaled_kernel`, :114-126)
//
// The quotient x / s is the multiply-and-correct quant_div (whose codes equal those of the
// correctly rounded division for every bf16 x with |x| <= amax) or, for a non-finite amax, the
// IEEE division; e4m3fn rounding is round-to-nearest-even, so the codes equal a CPU
// `(x / s).clamp(...).to(torch.float8_e4m3fn)` bit for bit.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.h"

namespace vdnh3 {
namespace {

__device__ __forceinline__ float absmax8(u32x4_t v, float m) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    m = fmaxf(m, fabsf(__uint_as_float(v[j] << 16)));
    m = fmaxf(m, fabsf(__uint_as_float(v[j] & 0xffff0000u)));
  }
  return m;
}

// The int8 (KIND 1) or e4m3fn (KIND 2) codes of the eight bf16 values of v divided by s, bytes
// in element order: quant_div with r = 1 / s, or the IEEE division when EXACT (non-finite amax).
template <int KIND, bool EXACT>
__device__ __forceinline__ u32x2_t codes8(u32x4_t v, float s, float r) {
  uint32_t w[2] = {0, 0};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float x0 = __uint_as_float(v[j] << 16), x1 = __uint_as_float(v[j] & 0xffff0000u);
    const float e0 = EXACT ? x0 / s : quant_div(x0, s, r), e1 = EXACT ? x1 / s : quant_div(x1, s, r);
    const uint32_t c0 = KIND == 1 ? i8_code(e0) : e4m3_code(fminf(fmaxf(e0, -kF8Max), kF8Max));
    const uint32_t c1 = KIND == 1 ? i8_code(e1) : e4m3_code(fminf(fmaxf(e1, -kF8Max), kF8Max));
    w[j >> 1] |= (c0 | (c1 << 8)) << (16 * (j & 1));
  }
  return u32x2_t{w[0], w[1]};
}

// One wavefront per row (4 rows per 256-thread workgroup). NCH > 0 (K <= 512 NCH): each lane
// loads its (up to NCH) 16-byte chunks of the row at once and keeps them in registers from the
// amax to the codes, so the row is read once with all its loads in flight. NCH == 0 (longer
// rows): two sweeps, the amax and then the codes (the second sweep served from L2).
template <int KIND, int NCH>
__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t *__restrict__ x, int64_t ldx, int M, int K,
                                                         uint8_t *__restrict__ q, int64_t ldq,
                                                         float *__restrict__ scale) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= M) return;
  const uint16_t *xr = x + (int64_t)row * ldx;
  const int chunks = K / 8;
  u32x4_t xv[NCH > 0 ? NCH : 1];
  float amax = 0.f;
  if constexpr (NCH > 0) {
#pragma unroll
    for (int u = 0; u < NCH; ++u) {
      const int c = lane + 64 * u;
      xv[u] = c < chunks ? ld16(xr + 8 * c) : u32x4_t{0, 0, 0, 0};  // zeros leave the amax alone
    }
#pragma unroll
    for (int u = 0; u < NCH; ++u) amax = absmax8(xv[u], amax);
  } else {
    for (int c = lane; c < chunks; c += 64) amax = absmax8(ld16(xr + 8 * c), amax);
  }
  amax = wave_max(amax);
  const float s = fmaxf(amax / (KIND == 1 ? kI8Max : kF8Max), 1e-12f), r = 1.f / s;
  if (lane == 0) scale[row] = s;
  uint8_t *qr = q + (int64_t)row * ldq;
  auto sweep = [&](auto exact) __device__ {
    constexpr bool E = decltype(exact)::value;
    if constexpr (NCH > 0) {
#pragma unroll
      for (int u = 0; u < NCH; ++u) {
        const int c = lane + 64 * u;
        if (c < chunks) *reinterpret_cast<u32x2_t *>(qr + 8 * c) = codes8<KIND, E>(xv[u], s, r);
      }
    } else {
      for (int c = lane; c < chunks; c += 64)
        *reinterpret_cast<u32x2_t *>(qr + 8 * c) = codes8<KIND, E>(ld16(xr + 8 * c), s, r);
    }
  };
  if (__builtin_isfinite(amax)) sweep(std::false_type{});
  else sweep(std::true_type{});
}

// The register-resident form with the fewest chunks per lane that holds the row (K <= 2048, 5120,
// 8192; more chunks cost registers and occupancy), else the two-sweep form.
template <int KIND>
void launch_quant_rows(dim3 grid, hipStream_t s, const uint16_t *x, int64_t ldx, int M, int K, uint8_t *q, int64_t ldq,
                       float *scale) {
  if (K <= 512 * 4)
    hipLaunchKernelGGL((quant_rows_kernel<KIND, 4>), grid, dim3(256), 0, s, x, ldx, M, K, q, ldq, scale);
  else if (K <= 512 * 10)
    hipLaunchKernelGGL((quant_rows_kernel<KIND, 10>), grid, dim3(256), 0, s, x, ldx, M, K, q, ldq, scale);
  else if (K <= 512 * 16)
    hipLaunchKernelGGL((quant_rows_kernel<KIND, 16>), grid, dim3(256), 0, s, x, ldx, M, K, q, ldq, scale);
  else
    hipLaunchKernelGGL((quant_rows_kernel<KIND, 0>), grid, dim3(256), 0, s, x, ldx, M, K, q, ldq, scale);
}

__global__ void fill_f32_kernel(float *p, float v) { *p = v; }

// Grid reduction of |x| into *amax (non-negative floats order like their bit patterns).
__global__ __launch_bounds__(256) void absmax_kernel(const uint16_t *__restrict__ x, int64_t n8,
                                                     float *__restrict__ amax) {
  __shared__ float red[4];
  float m = 0.f;
  for (int64_t c = blockIdx.x * 256 + threadIdx.x; c < n8; c += (int64_t)gridDim.x * 256) {
    const u32x4_t v = ld16(x + 8 * c);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      m = fmaxf(m, fabsf(__uint_as_float(v[j] << 16)));
      m = fmaxf(m, fabsf(__uint_as_float(v[j] & 0xffff0000u)));
    }
  }
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    atomicMax(reinterpret_cast<unsigned int *>(amax), __float_as_uint(m));
  }
}

__global__ __launch_bounds__(256) void cast_tensor_f8_kernel(const uint16_t *__restrict__ x, int64_t n8,
                                                             const float *__restrict__ amax, uint8_t *__restrict__ q,
                                                             float *__restrict__ scale) {
  const float a = *amax, s = fmaxf(a / kF8Max, 1e-12f), r = 1.f / s;
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale = s;
  auto sweep = [&](auto exact) __device__ {
    for (int64_t c = blockIdx.x * 256 + threadIdx.x; c < n8; c += (int64_t)gridDim.x * 256)
      *reinterpret_cast<u32x2_t *>(q + 8 * c) = codes8<2, decltype(exact)::value>(ld16(x + 8 * c), s, r);
  };
  if (__builtin_isfinite(a)) sweep(std::false_type{});
  else sweep(std::true_type{});
}

// ---------------------------------------------------------------------------------
// Allocation-free per-tensor fp8 quantisation (vdnh3_quant_tensor_f8_noalloc). The amax is
// reduced in two deterministic levels through a file-scope device array instead of a caller
// workspace: one partial maximum per span of kAmaxSpan elements (one workgroup each), then one
// workgroup reduces the partials into slot kAmaxPartials, which the cast pass reads. Every slot a
// call reads is written by that call, so nothing needs clearing; calls that overlap on one GPU
// share the array and race.
constexpr int kAmaxSpanChunks = 2048;                  // 16-byte chunks per partial (8 per thread)
constexpr int64_t kAmaxSpan = 8 * kAmaxSpanChunks;     // 16,384 elements per partial maximum
constexpr int kAmaxPartials = 16384;                   // n <= kAmaxSpan * kAmaxPartials (268,435,456)
constexpr int kScratchFloats = kAmaxPartials + 64;     // partials, then the total (64 KiB + 256 B)
__device__ __align__(256) float scratch[kScratchFloats];

__device__ __forceinline__ float block_max256(float m, float *red) {
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// partial[b] = max |x| over chunks [b * kAmaxSpanChunks, (b + 1) * kAmaxSpanChunks) (clipped to n8)
__global__ __launch_bounds__(256) void absmax_partial_kernel(const uint16_t *__restrict__ x, int64_t n8,
                                                             float *__restrict__ partial) {
  __shared__ float red[4];
  const int64_t c0 = (int64_t)blockIdx.x * kAmaxSpanChunks;
  const int64_t c1 = c0 + kAmaxSpanChunks < n8 ? c0 + kAmaxSpanChunks : n8;
  float m = 0.f;
  for (int64_t c = c0 + threadIdx.x; c < c1; c += 256) m = absmax8(ld16(x + 8 * c), m);
  m = block_max256(m, red);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// *total = max over partial[0 .. count)
__global__ __launch_bounds__(256) void absmax_total_kernel(const float *__restrict__ partial, int count,
                                                           float *__restrict__ total) {
  __shared__ float red[4];
  float m = 0.f;
  for (int i = threadIdx.x; i < count; i += 256) m = fmaxf(m, partial[i]);
  m = block_max256(m, red);
  if (threadIdx.x == 0) *total = m;
}

// Device address of `scratch` on the device `stream` runs on (the current device for the null
// stream), looked up once per device with that device current: each GPU holds its own copy of the
// array. The array's name is a host-side handle only; every kernel argument uses this address.
int scratch_address(hipStream_t stream, float **out) {
  constexpr int kMaxDevices = 64;
  static std::mutex lock;
  static float *addr[kMaxDevices] = {};
  int current = 0;
  hipError_t err = hipGetDevice(&current);
  if (err != hipSuccess) return set_error(VDNH3_ERR_RUNTIME, "no current HIP device: %s", hipGetErrorString(err));
  hipDevice_t dev = current;
  if (stream != nullptr && (err = hipStreamGetDevice(stream, &dev)) != hipSuccess)
    return set_error(VDNH3_ERR_RUNTIME, "hipStreamGetDevice failed: %s", hipGetErrorString(err));
  VDNH3_HOST_CHECK(dev >= 0 && dev < kMaxDevices, VDNH3_ERR_RUNTIME, "device %d is beyond the %d this library tracks",
                   (int)dev, kMaxDevices);
  std::lock_guard<std::mutex> guard(lock);
  if (addr[dev] == nullptr) {
    if (dev != current && (err = hipSetDevice(dev)) != hipSuccess)
      return set_error(VDNH3_ERR_RUNTIME, "hipSetDevice(%d) failed: %s", (int)dev, hipGetErrorString(err));
    void *p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != current) (void)hipSetDevice(current);
    if (err != hipSuccess || p == nullptr)
      return set_error(VDNH3_ERR_RUNTIME, "hipGetSymbolAddress(scratch) on device %d failed: %s", (int)dev,
                       hipGetErrorString(err));
    addr[dev] = static_cast<float *>(p);
  }
  *out = addr[dev];
  return VDNH3_OK;
}

}  // namespace
}  // namespace vdnh3

extern "C" int vdnh3_quant_rows(int kind, const uint16_t *x, int64_t ldx, int M, int K, uint8_t *q, int64_t ldq,
                                float *scale, void *stream) {
  using namespace vdnh3;
  VDNH3_HOST_CHECK(kind == 1 || kind == 2, VDNH3_ERR_INVALID, "quant_rows: kind must be 1 (int8) or 2 (fp8)");
  VDNH3_HOST_CHECK(x && q && scale && M > 0 && K > 0, VDNH3_ERR_INVALID, "quant_rows: empty or null operand");
  VDNH3_HOST_CHECK(K % 8 == 0 && ldx % 8 == 0 && ldq % 8 == 0 && ldx >= K && ldq >= K, VDNH3_ERR_INVALID,
                   "quant_rows: K and leading dimensions must be multiples of 8 covering K");
  VDNH3_HOST_CHECK(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 8 == 0,
                   VDNH3_ERR_INVALID, "quant_rows: x must be 16-byte and q 8-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((M + 3) / 4);
  if (kind == 1)
    launch_quant_rows<1>(grid, s, x, ldx, M, K, q, ldq, scale);
  else
    launch_quant_rows<2>(grid, s, x, ldx, M, K, q, ldq, scale);
  return check_launch("quant_rows");
}

extern "C" int vdnh3_quant_tensor_f8(const uint16_t *x, int64_t n, uint8_t *q, float *scale, float *amax_workspace,
                                     void *stream) {
  using namespace vdnh3;
  VDNH3_HOST_CHECK(x && q && scale && amax_workspace && n > 0, VDNH3_ERR_INVALID,
                   "quant_tensor_f8: empty or null operand");
  VDNH3_HOST_CHECK(n % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 8 == 0,
                   VDNH3_ERR_INVALID, "quant_tensor_f8: n must be a multiple of 8, x 16-byte and q 8-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n8 = n / 8;
  const int blocks = (int)std::min<int64_t>((n8 + 255) / 256, 4096);
  hipLaunchKernelGGL(fill_f32_kernel, dim3(1), dim3(1), 0, s, amax_workspace, 0.f);
  hipLaunchKernelGGL(absmax_kernel, dim3(blocks), dim3(256), 0, s, x, n8, amax_workspace);
  hipLaunchKernelGGL(cast_tensor_f8_kernel, dim3(blocks), dim3(256), 0, s, x, n8, amax_workspace, q, scale);
  return check_launch("quant_tensor_f8");
}

extern "C" size_t vdnh3_quant_tensor_f8_noalloc_max_elements(void) {
  return (size_t)vdnh3::kAmaxSpan * (size_t)vdnh3::kAmaxPartials;
}

extern "C" int vdnh3_quant_tensor_f8_noalloc(const uint16_t *x, int64_t n, uint8_t *q, float *scale, void *stream) {
  using namespace vdnh3;
  VDNH3_HOST_CHECK(x && q && scale && n > 0, VDNH3_ERR_INVALID, "quant_tensor_f8_noalloc: empty or null operand");
  VDNH3_HOST_CHECK(n % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 8 == 0,
                   VDNH3_ERR_INVALID,
                   "quant_tensor_f8_noalloc: n must be a multiple of 8, x 16-byte and q 8-byte aligned");
  VDNH3_HOST_CHECK(n <= kAmaxSpan * kAmaxPartials, VDNH3_ERR_INVALID,
                   "quant_tensor_f8_noalloc: %lld elements exceed the %lld its fixed scratch (%d partial maxima of "
                   "%lld elements) supports; use vdnh3_quant_tensor_f8 with a workspace",
                   (long long)n, (long long)(kAmaxSpan * kAmaxPartials), kAmaxPartials, (long long)kAmaxSpan);
  hipStream_t s = static_cast<hipStream_t>(stream);
  float *buf = nullptr;
  const int rc = scratch_address(s, &buf);
  if (rc) return rc;
  const int64_t n8 = n / 8;
  const int partials = (int)((n8 + kAmaxSpanChunks - 1) / kAmaxSpanChunks);
  const int blocks = (int)std::min<int64_t>((n8 + 255) / 256, 4096);
  hipLaunchKernelGGL(absmax_partial_kernel, dim3(partials), dim3(256), 0, s, x, n8, buf);
  hipLaunchKernelGGL(absmax_total_kernel, dim3(1), dim3(256), 0, s, buf, partials, buf + kAmaxPartials);
  hipLaunchKernelGGL(cast_tensor_f8_kernel, dim3(blocks), dim3(256), 0, s, x, n8, buf + kAmaxPartials, q, scale);
  return check_launch("quant_tensor_f8_noalloc");
}
