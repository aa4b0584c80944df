// Pointwise passes of the MiniMax-H3 DiT block around attention and the MLP on gfx950
// (HBM-bound), the fused stretches of vdn_h3/block_kernels.py:
//
//   rmsnorm_modulate : h = (rms_norm(x, w, eps) * (1 + scale[seg]) + shift[seg])      (:85-89)
//   gated_residual   : x' = x + gate[seg] * branch                                    (:92-93)
//   swiglu           : a = silu(hidden[:, :F]) * hidden[:, F:]                         (:113-116)
//   swiglu_quant     : the row-wise int8 / fp8 activation quantisation of a (the input of the
//                      W8A8 fc2), without materialising a
//
// seg = idx[row] selects the modulation row of that token (the AdaLN segment map of
// BlockPointwiseCache, vdn_h3/block_kernels.py:25-82). The arithmetic follows the reference's
// torch ops in bf16: every op's result is rounded to bf16 (rms_norm once, then 1 + scale,
// the product, the sum; silu, then the product), so a CPU evaluation of the same expressions
// gives the same bits.
#include <type_traits>

#include "common.h"

namespace vdnh3 {
namespace {

__device__ __forceinline__ void unpack8f(u32x4_t w, float *x) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t u = w[j >> 1];
    x[j] = __uint_as_float((j & 1) ? (u & 0xffff0000u) : (u << 16));
  }
}

__device__ __forceinline__ u32x4_t pack8f(const float *y) {
  return u32x4_t{pack_bf2(y[0], y[1]), pack_bf2(y[2], y[3]), pack_bf2(y[4], y[5]), pack_bf2(y[6], y[7])};
}

// 8 modulation values (bf16, or fp32 rounded to bf16 like the reference's .to(bf16)) at p[c]
__device__ __forceinline__ void load_mod8(const void *p, int64_t off, int bf16, float *v) {
  if (bf16) {
    unpack8f(ld16(static_cast<const uint16_t *>(p) + off), v);
  } else {
    const f32x4_t a = *reinterpret_cast<const f32x4_t *>(static_cast<const float *>(p) + off);
    const f32x4_t b = *reinterpret_cast<const f32x4_t *>(static_cast<const float *>(p) + off + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = round_bf(a[j]);
      v[4 + j] = round_bf(b[j]);
    }
  }
}

template <int NW>
__device__ __forceinline__ float block_max(float v, float *red) {
  v = wave_max(v);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) m = fmaxf(m, red[i]);
  return m;
}

__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) s += red[w];
  return s;
}

// 8 channels per thread per pass of a 256-thread workgroup; a row stays in registers between the
// sum of squares and the output (hidden <= 8 * 256 * kRowChunks).
constexpr int kRowChunks = 4;
constexpr int kNormGroups = 768;  // workgroups of rmsnorm_modulate: three per CU (132 VGPRs)

// A workgroup walks a contiguous block of rows: the weight row stays in registers (packed bf16),
// and so do the segment's 1 + scale and shift (bf16, as the reference rounds them) while
// consecutive rows share a segment; the next row's x is in flight while the current row is reduced
// and written, with one barrier per row (two reduction slots). A thread's chunks and the reduction
// order are those of a one-row workgroup, so every row gets the same bits either way.
__global__ __launch_bounds__(256) void rmsnorm_modulate_kernel(
    const uint16_t *__restrict__ x, int64_t x_row, const uint16_t *__restrict__ w, float eps,
    const void *__restrict__ scale, const void *__restrict__ shift, int64_t mod_row, int mod_bf16,
    const int32_t *__restrict__ idx, int table_rows, uint16_t *__restrict__ out, int64_t out_row, int hidden,
    int rows, int rows_per_group) {
  __shared__ float red[2][4];
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_group;
  const int64_t r1 = r0 + rows_per_group < rows ? r0 + rows_per_group : rows;
  const int chunks = hidden / 8, tid = threadIdx.x;
  u32x4_t wv[kRowChunks], opsc[kRowChunks], shv[kRowChunks], xa[kRowChunks], xb[kRowChunks];
#pragma unroll
  for (int u = 0; u < kRowChunks; ++u) {
    const int c = tid + 256 * u;
    wv[u] = c < chunks ? ld16(w + 8 * c) : u32x4_t{0, 0, 0, 0};
    opsc[u] = shv[u] = u32x4_t{0, 0, 0, 0};
  }
  int cur = -1;  // the segment whose modulation the registers hold (none yet)
  bool cur_ok = false;
  auto load_x = [&](int64_t row, u32x4_t (&xv)[kRowChunks]) __device__ {
#pragma unroll
    for (int u = 0; u < kRowChunks; ++u) {
      const int c = tid + 256 * u;
      if (c < chunks) xv[u] = ld16(x + row * x_row + 8 * c);
    }
  };
  auto process = [&](int64_t row, const u32x4_t (&xv)[kRowChunks], float *slot) __device__ {
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < kRowChunks; ++u) {
      if (tid + 256 * u < chunks) {
        float v[8];
        unpack8f(xv[u], v);
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = fmaf(v[j], v[j], ss);
      }
    }
    // a segment index outside the modulation table reads row 0 and writes a NaN row instead of
    // reading past the table
    const int seg = idx[row];
    if (seg != cur || cur < 0) {
      cur = seg;
      cur_ok = (unsigned)seg < (unsigned)table_rows;
      const int64_t mrow = (int64_t)(cur_ok ? seg : 0) * mod_row;
#pragma unroll
      for (int u = 0; u < kRowChunks; ++u) {
        const int c = tid + 256 * u;
        if (c >= chunks) continue;
        float sc[8], sh[8];
        load_mod8(scale, mrow + 8 * c, mod_bf16, sc);
        load_mod8(shift, mrow + 8 * c, mod_bf16, sh);
#pragma unroll
        for (int j = 0; j < 8; ++j) sc[j] = 1.f + sc[j];
        opsc[u] = pack8f(sc);  // bf16(1 + scale), the reference's rounding
        shv[u] = pack8f(sh);   // already bf16 values: exact
      }
    }
    const float r = 1.f / sqrtf(block_sum(ss, slot) / (float)hidden + eps);
#pragma unroll
    for (int u = 0; u < kRowChunks; ++u) {
      const int c = tid + 256 * u;
      if (c >= chunks) continue;
      float v[8], wf[8], o[8], sh[8], y[8];
      unpack8f(xv[u], v);  // the row is still in registers, packed
      unpack8f(wv[u], wf);
      unpack8f(opsc[u], o);
      unpack8f(shv[u], sh);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float n = round_bf(v[j] * r * wf[j]);  // F.rms_norm, one rounding
        const float p = round_bf(n * o[j]);
        y[j] = cur_ok ? p + sh[j] : __builtin_nanf("");
      }
      st16(out + row * out_row + 8 * c, pack8f(y));
    }
  };
  // two rows per trip, so both x buffers have fixed names
  load_x(r0, xa);
  for (int64_t row = r0; row < r1; row += 2) {
    if (row + 1 < r1) load_x(row + 1, xb);
    process(row, xa, red[0]);
    if (row + 1 >= r1) break;
    if (row + 2 < r1) load_x(row + 2, xa);
    process(row + 1, xb, red[1]);
  }
}

// x' = bf16(x + bf16(bf16(gate[seg]) * branch)); 8 channels per thread, any number of rows
__global__ __launch_bounds__(256) void gated_residual_kernel(
    const uint16_t *__restrict__ x, int64_t x_row, const void *__restrict__ gate, int64_t gate_row, int gate_bf16,
    const int32_t *__restrict__ idx, int table_rows, const uint16_t *__restrict__ b, int64_t b_row,
    uint16_t *__restrict__ out, int64_t out_row, int64_t rows, int chunks) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= rows * chunks) return;
  const int64_t row = t / chunks;
  const int c = (int)(t - row * chunks);
  float xv[8], bv[8], gv[8], y[8];
  unpack8f(ld16(x + row * x_row + 8 * c), xv);
  unpack8f(ld16(b + row * b_row + 8 * c), bv);
  const int seg = idx[row];
  const bool seg_ok = (unsigned)seg < (unsigned)table_rows;  // else row 0 is read and NaN written
  load_mod8(gate, (int64_t)(seg_ok ? seg : 0) * gate_row + 8 * c, gate_bf16, gv);
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = seg_ok ? xv[j] + round_bf(gv[j] * bv[j]) : __builtin_nanf("");
  st16(out + row * out_row + 8 * c, pack8f(y));
}

// a = bf16(bf16(silu(g)) * u) for 8 channels of one row
__device__ __forceinline__ void swiglu8(const uint16_t *hr, int ffn, int c, float *a) {
  float g[8], u[8];
  unpack8f(ld16(hr + 8 * c), g);
  unpack8f(ld16(hr + ffn + 8 * c), u);
#pragma unroll
  for (int j = 0; j < 8; ++j) a[j] = round_bf(silu_bf(g[j]) * u[j]);
}

__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t *__restrict__ h, int64_t h_row, int ffn,
                                                     uint16_t *__restrict__ out, int64_t out_row, int64_t rows) {
  const int chunks = ffn / 8;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= rows * chunks) return;
  const int64_t row = t / chunks;
  const int c = (int)(t - row * chunks);
  float a[8];
  swiglu8(h + row * h_row, ffn, c, a);
  st16(out + row * out_row + 8 * c, pack8f(a));
}

// For ffn > 8 * kQuantThreads * kQuantChunks: one wavefront per row, like quant_rows: amax of a over
// the row, then the codes (the second sweep recomputes a from the fc1 output, served from L2).
// scale[row] = max(amax / qmax, 1e-12).
template <int KIND>
__global__ __launch_bounds__(256) void swiglu_quant_kernel(const uint16_t *__restrict__ h, int64_t h_row, int rows,
                                                           int ffn, uint8_t *__restrict__ q, int64_t q_row,
                                                           float *__restrict__ scale) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  const uint16_t *hr = h + (int64_t)row * h_row;
  const int chunks = ffn / 8;
  float amax = 0.f;
  for (int c = lane; c < chunks; c += 64) {
    float a[8];
    swiglu8(hr, ffn, c, a);
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(a[j]));
  }
  amax = wave_max(amax);
  const float s = fmaxf(amax / (KIND == 1 ? kI8Max : kF8Max), 1e-12f), r = 1.f / s;
  if (lane == 0) scale[row] = s;
  uint8_t *qr = q + (int64_t)row * q_row;
  // the codes of a / s (quant_div for a finite amax, the division otherwise)
  auto sweep = [&](auto exact) __device__ {
    for (int c = lane; c < chunks; c += 64) {
      float a[8];
      swiglu8(hr, ffn, c, a);
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float e = decltype(exact)::value ? a[j] / s : quant_div(a[j], s, r);
        const uint32_t code = KIND == 1 ? i8_code(e) : e4m3_code(fminf(fmaxf(e, -kF8Max), kF8Max));
        if (j < 4)
          lo |= code << (8 * j);
        else
          hi |= code << (8 * (j - 4));
      }
      *reinterpret_cast<u32x2_t *>(qr + 8 * c) = u32x2_t{lo, hi};
    }
  };
  if (__builtin_isfinite(amax)) sweep(std::false_type{});
  else sweep(std::true_type{});
}

// One workgroup of kQuantThreads threads per row for ffn <= 8 * kQuantThreads * kQuantChunks (16,384):
// each thread loads all its chunks of g and u up front, keeps a = bf16(silu(g) * u) as packed bf16
// between the row's amax and the codes, so the fc1 output is read once. Same arithmetic as
// swiglu_quant_kernel. 512 threads per row measured faster than 256 or 1024.
constexpr int kQuantThreads = 512, kQuantChunks = 4;

template <int KIND>
__global__ __launch_bounds__(kQuantThreads) void swiglu_quant_row_kernel(const uint16_t *__restrict__ h,
                                                                         int64_t h_row,
                                                               int ffn, uint8_t *__restrict__ q, int64_t q_row,
                                                               float *__restrict__ scale) {
  __shared__ float red[kQuantThreads / 64];
  const int64_t row = blockIdx.x;
  const uint16_t *hr = h + row * h_row;
  const int chunks = ffn / 8;
  u32x4_t gr[kQuantChunks], ur[kQuantChunks];
#pragma unroll
  for (int u = 0; u < kQuantChunks; ++u) {
    const int c = threadIdx.x + kQuantThreads * u;
    if (c < chunks) {
      gr[u] = ld16(hr + 8 * c);
      ur[u] = ld16(hr + ffn + 8 * c);
    }
  }
  u32x4_t a[kQuantChunks];
  float amax = 0.f;
#pragma unroll
  for (int u = 0; u < kQuantChunks; ++u) {
    const int c = threadIdx.x + kQuantThreads * u;
    if (c >= chunks) continue;
    float g[8], uv[8], av[8];
    unpack8f(gr[u], g);
    unpack8f(ur[u], uv);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      av[j] = round_bf(silu_bf(g[j]) * uv[j]);
      amax = fmaxf(amax, fabsf(av[j]));
    }
    a[u] = pack8f(av);  // exact: av holds bf16 values
  }
  amax = block_max<kQuantThreads / 64>(amax, red);
  const float s = fmaxf(amax / (KIND == 1 ? kI8Max : kF8Max), 1e-12f), r = 1.f / s;
  if (threadIdx.x == 0) scale[row] = s;
  uint8_t *qr = q + row * q_row;
  // the codes of a / s (quant_div for a finite amax, the division otherwise)
  auto sweep = [&](auto exact) __device__ {
#pragma unroll
    for (int u = 0; u < kQuantChunks; ++u) {
      const int c = threadIdx.x + kQuantThreads * u;
      if (c >= chunks) continue;
      float av[8];
      unpack8f(a[u], av);
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float e = decltype(exact)::value ? av[j] / s : quant_div(av[j], s, r);
        const uint32_t code = KIND == 1 ? i8_code(e) : e4m3_code(fminf(fmaxf(e, -kF8Max), kF8Max));
        if (j < 4)
          lo |= code << (8 * j);
        else
          hi |= code << (8 * (j - 4));
      }
      *reinterpret_cast<u32x2_t *>(qr + 8 * c) = u32x2_t{lo, hi};
    }
  };
  if (__builtin_isfinite(amax)) sweep(std::false_type{});
  else sweep(std::true_type{});
}

int check_vec8(const void *p, int64_t row, const char *name, int esize = 2) {
  VDNH3_HOST_CHECK(p != nullptr, VDNH3_ERR_INVALID, "%s is null", name);
  VDNH3_HOST_CHECK((row * esize) % 16 == 0 && reinterpret_cast<uintptr_t>(p) % 16 == 0, VDNH3_ERR_INVALID,
                   "%s must be 16-byte aligned with a row stride of a multiple of 16 bytes", name);
  return VDNH3_OK;
}

}  // namespace
}  // namespace vdnh3

using vdnh3::check_vec8;

extern "C" int vdnh3_rmsnorm_modulate(const uint16_t *x, int64_t x_row, const uint16_t *weight, float eps,
                                      const void *scale, const void *shift, int64_t mod_row, int mod_bf16,
                                      const int32_t *idx, int table_rows, uint16_t *out, int64_t out_row, int rows,
                                      int hidden, void *stream) {
  VDNH3_HOST_CHECK(rows > 0 && hidden > 0 && hidden % 8 == 0 && hidden <= 8 * 256 * vdnh3::kRowChunks,
                   VDNH3_ERR_INVALID, "rmsnorm_modulate: hidden must be a positive multiple of 8 up to %d, got %d",
                   8 * 256 * vdnh3::kRowChunks, hidden);
  int rc = check_vec8(x, x_row, "x");
  if (!rc) rc = check_vec8(out, out_row, "out");
  if (!rc) rc = check_vec8(weight, 0, "weight");
  if (!rc) rc = check_vec8(scale, mod_row, "scale", mod_bf16 ? 2 : 4);
  if (!rc) rc = check_vec8(shift, mod_row, "shift", mod_bf16 ? 2 : 4);
  if (rc) return rc;
  VDNH3_HOST_CHECK(idx != nullptr && table_rows > 0, VDNH3_ERR_INVALID,
                   "rmsnorm_modulate: null segment index or empty modulation table");
  const int per = (rows + vdnh3::kNormGroups - 1) / vdnh3::kNormGroups, groups = (rows + per - 1) / per;
  hipLaunchKernelGGL(vdnh3::rmsnorm_modulate_kernel, dim3(groups), dim3(256), 0, static_cast<hipStream_t>(stream),
                     x, x_row, weight, eps, scale, shift, mod_row, mod_bf16, idx, table_rows, out, out_row, hidden,
                     rows, per);
  return vdnh3::check_launch("rmsnorm_modulate");
}

extern "C" int vdnh3_gated_residual(const uint16_t *x, int64_t x_row, const void *gate, int64_t gate_row,
                                    int gate_bf16, const int32_t *idx, int table_rows, const uint16_t *branch,
                                    int64_t branch_row,
                                    uint16_t *out, int64_t out_row, int rows, int hidden, void *stream) {
  VDNH3_HOST_CHECK(rows > 0 && hidden > 0 && hidden % 8 == 0, VDNH3_ERR_INVALID,
                   "gated_residual: hidden must be a positive multiple of 8, got %d", hidden);
  int rc = check_vec8(x, x_row, "x");
  if (!rc) rc = check_vec8(branch, branch_row, "branch");
  if (!rc) rc = check_vec8(out, out_row, "out");
  if (!rc) rc = check_vec8(gate, gate_row, "gate", gate_bf16 ? 2 : 4);
  if (rc) return rc;
  VDNH3_HOST_CHECK(idx != nullptr && table_rows > 0, VDNH3_ERR_INVALID,
                   "gated_residual: null segment index or empty modulation table");
  const int chunks = hidden / 8;
  const int64_t threads = (int64_t)rows * chunks;
  hipLaunchKernelGGL(vdnh3::gated_residual_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, x_row, gate, gate_row, gate_bf16, idx, table_rows, branch,
                     branch_row,
                     out, out_row, (int64_t)rows, chunks);
  return vdnh3::check_launch("gated_residual");
}

extern "C" int vdnh3_swiglu(const uint16_t *h, int64_t h_row, int rows, int ffn, uint16_t *out, int64_t out_row,
                            void *stream) {
  VDNH3_HOST_CHECK(rows > 0 && ffn > 0 && ffn % 8 == 0, VDNH3_ERR_INVALID,
                   "swiglu: the half width must be a positive multiple of 8, got %d", ffn);
  int rc = check_vec8(h, h_row, "hidden");
  if (!rc) rc = check_vec8(out, out_row, "out");
  if (rc) return rc;
  const int64_t threads = (int64_t)rows * (ffn / 8);
  hipLaunchKernelGGL(vdnh3::swiglu_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), h, h_row, ffn, out, out_row, (int64_t)rows);
  return vdnh3::check_launch("swiglu");
}

extern "C" int vdnh3_swiglu_quant_rows(int kind, const uint16_t *h, int64_t h_row, int rows, int ffn, uint8_t *q,
                                       int64_t q_row, float *scale, void *stream) {
  VDNH3_HOST_CHECK(kind == 1 || kind == 2, VDNH3_ERR_INVALID, "swiglu_quant_rows: kind must be 1 (int8) or 2 (fp8)");
  VDNH3_HOST_CHECK(rows > 0 && ffn > 0 && ffn % 8 == 0, VDNH3_ERR_INVALID,
                   "swiglu_quant_rows: the half width must be a positive multiple of 8, got %d", ffn);
  int rc = check_vec8(h, h_row, "hidden");
  if (rc) return rc;
  VDNH3_HOST_CHECK(q && scale && q_row % 8 == 0 && reinterpret_cast<uintptr_t>(q) % 8 == 0, VDNH3_ERR_INVALID,
                   "swiglu_quant_rows: codes must be 8-byte aligned with a row stride of a multiple of 8");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (ffn <= 8 * vdnh3::kQuantThreads * vdnh3::kQuantChunks) {
    if (kind == 1)
      hipLaunchKernelGGL(vdnh3::swiglu_quant_row_kernel<1>, dim3(rows), dim3(vdnh3::kQuantThreads), 0, s, h, h_row,
                         ffn, q, q_row,
                         scale);
    else
      hipLaunchKernelGGL(vdnh3::swiglu_quant_row_kernel<2>, dim3(rows), dim3(vdnh3::kQuantThreads), 0, s, h, h_row,
                         ffn, q, q_row,
                         scale);
    return vdnh3::check_launch("swiglu_quant_rows");
  }
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (kind == 1)
    hipLaunchKernelGGL(vdnh3::swiglu_quant_kernel<1>, grid, dim3(256), 0, s, h, h_row, rows, ffn, q, q_row, scale);
  else
    hipLaunchKernelGGL(vdnh3::swiglu_quant_kernel<2>, grid, dim3(256), 0, s, h, h_row, rows, ffn, q, q_row, scale);
  return vdnh3::check_launch("swiglu_quant_rows");
}
