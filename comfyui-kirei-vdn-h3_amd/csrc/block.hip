// Pointwise passes of the hybrid attention block on gfx950 (HBM-bound):
//
//   qk_rmsnorm : the block's q_norm / k_norm over the head dim (vdn_h3/hybrid.py:271-273 with
//                rope_freqs=None), y = bf16(x * rsqrt(mean(x^2) + eps) * w), fp32 statistics,
//                written to separate normalised copies (the VDN branch reads the raw q / k);
//                with rope_freqs (vdn_h3/hybrid.py:274-292, the fused RMSNorm + split-half RoPE
//                the reference calls), the normalised fp32 vector y is rotated before its one
//                rounding: for i < rot/2 the pair (y_i, y_{i+rot/2}) becomes F_i (y_i, y_{i+rot/2})
//                with F_i the row's 2x2 matrix [[f00, f01], [f10, f11]]; channels >= rot pass;
//   head_gate  : apply_softmax_gate (vdn_h3/softmax_kernels.py:8-9), out = bf16(O * g) per
//                (row, head), flattened to [S, H*D].
//
// Both kernels give each head vector to 16 lanes x 16 bytes (D = 128) or 8 lanes (D = 64): a
// wavefront covers 4 (8) head vectors of one row with fully coalesced 16-byte accesses, and the
// sum of squares is reduced with lane shuffles inside the lane group.
#include "common.h"
#include "qk_norm.h"

namespace vdnh3 {
namespace {

__device__ __forceinline__ void unpack8(u32x4_t w, float *x) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t u = w[j >> 1];
    x[j] = __uint_as_float((j & 1) ? (u & 0xffff0000u) : (u << 16));
  }
}

__device__ __forceinline__ u32x4_t pack8(const float *y) {
  return u32x4_t{pack_bf2(y[0], y[1]), pack_bf2(y[2], y[3]), pack_bf2(y[4], y[5]), pack_bf2(y[6], y[7])};
}

// One thread = 8 consecutive channels of one head vector. vec indexes (row, which, head) with
// which = 0 for q, 1 for k; grid covers seq * 2 * heads vectors (the plain norm: one vector per lane
// group is faster here than the row walk below, 0.30 against 0.32 ms at 40 688 x 40 x 128).
template <int D>
__global__ __launch_bounds__(256) void qk_rmsnorm_kernel(const uint16_t *__restrict__ q, int64_t q_row,
                                                         int64_t q_head, const uint16_t *__restrict__ k,
                                                         int64_t k_row, int64_t k_head,
                                                         const uint16_t *__restrict__ wq,
                                                         const uint16_t *__restrict__ wk, float q_eps,
                                                         float k_eps, uint16_t *__restrict__ qo, int64_t qo_row,
                                                         int64_t qo_head, uint16_t *__restrict__ ko, int64_t ko_row,
                                                         int64_t ko_head, int64_t n_vec, int heads) {
  constexpr int LANES = D / 8;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t vec = t / LANES;
  const int c = (int)(t % LANES);
  if (vec >= n_vec) return;  // lane groups are aligned: a group is wholly in range or wholly out
  const int head = (int)(vec % heads);
  const int which = (int)((vec / heads) & 1);
  const int64_t row = vec / (2 * heads);
  const uint16_t *src = which ? k + row * k_row + head * k_head : q + row * q_row + head * q_head;
  uint16_t *dst = which ? ko + row * ko_row + head * ko_head : qo + row * qo_row + head * qo_head;
  float x[8], wf[8], y[8];
  unpack8(ld16(src + 8 * c), x);
  unpack8(ld16((which ? wk : wq) + 8 * c), wf);
  const float r = rms_factor(group_tree_sum<LANES>(chunk_sumsq(x)), D, which ? k_eps : q_eps);
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = x[j] * r * wf[j];
  st16(dst + 8 * c, pack8(y));
}

// The RMSNorm + split-half RoPE pass walks rows: a workgroup takes rows blockIdx.x, blockIdx.x + gridDim.x,
// ... and covers each row's 2 * heads vectors (q heads, then k heads) in passes of 256 / LANES vectors, the
// loads of up to RB passes issued before their arithmetic. Lane c of a vector's lane group holds channels
// 8c .. 8c + 7. Per row, the row's rot/2 rotation matrices are staged in LDS once (double-buffered, so one
// barrier per row; a table shared by every row is staged once); freqs element (row, i, r, c) sits at
// freqs[row * f_row + 4 i + 2 r + c]; the partner channel i +- rot/2 lives rot/16 lanes away in the same
// lane group.
template <int D>
__global__ __launch_bounds__(256) void qk_rmsnorm_rope_kernel(const uint16_t *__restrict__ q, int64_t q_row,
                                                              int64_t q_head, const uint16_t *__restrict__ k,
                                                              int64_t k_row, int64_t k_head,
                                                              const uint16_t *__restrict__ wq,
                                                              const uint16_t *__restrict__ wk, float q_eps,
                                                              float k_eps, const float *__restrict__ freqs,
                                                              int64_t f_row, int rot, uint16_t *__restrict__ qo,
                                                              int64_t qo_row, int64_t qo_head,
                                                              uint16_t *__restrict__ ko, int64_t ko_row,
                                                              int64_t ko_head, int seq, int heads) {
  constexpr int LANES = D / 8, VPW = 256 / LANES, RB = 4;
  __shared__ f32x4_t tab[2][D / 2];
  const int c = (int)threadIdx.x % LANES, v0 = (int)threadIdx.x / LANES;
  const int nv = 2 * heads;
  const int half = rot >> 1, step = half >> 3;  // rot is a multiple of 16 (host check)
  const bool first = 8 * c < half, rotated = 8 * c < rot;
  const int lane = __lane_id();
  const int partner = first ? lane + step : lane - step;
  const int i0 = first ? 8 * c : 8 * c - half;  // pair index of channel 8c
  float wqf[8], wkf[8];
  unpack8(ld16(wq + 8 * c), wqf);
  unpack8(ld16(wk + 8 * c), wkf);
  const bool shared = f_row == 0;
  if (shared) {
    if ((int)threadIdx.x < half) tab[0][threadIdx.x] = reinterpret_cast<const f32x4_t *>(freqs)[threadIdx.x];
    __syncthreads();
  }
  int b = 0;
  for (int64_t row = blockIdx.x; row < seq; row += gridDim.x) {
    if (!shared) {
      // buffer b was last read for row - 2 gridDim.x, before every thread passed the previous row's barrier
      if ((int)threadIdx.x < half)
        tab[b][threadIdx.x] = reinterpret_cast<const f32x4_t *>(freqs + row * f_row)[threadIdx.x];
      __syncthreads();
    }
    const f32x4_t *f = tab[shared ? 0 : b] + i0;
    for (int base = v0; base < nv; base += RB * VPW) {
      u32x4_t raw[RB];
#pragma unroll
      for (int u = 0; u < RB; ++u) {
        const int v = base + u * VPW;
        if (v < nv) {
          const int which = v >= heads, head = which ? v - heads : v;
          raw[u] = ld16((which ? k + row * k_row + head * k_head : q + row * q_row + head * q_head) + 8 * c);
        }
      }
#pragma unroll
      for (int u = 0; u < RB; ++u) {
        const int v = base + u * VPW;
        if (v >= nv) break;  // uniform over a lane group: its vectors are whole
        const int which = v >= heads, head = which ? v - heads : v;
        float x[8], y[8], o[8];
        unpack8(raw[u], x);
        const float r = rms_factor(group_tree_sum<LANES>(chunk_sumsq(x)), D, which ? k_eps : q_eps);
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = x[j] * r * (which ? wkf[j] : wqf[j]);
        if (D == 128 && rot == 128) {
          // full rotation: the partner is 8 lanes away inside the vector's 16-lane DPP row (row_ror:8)
#pragma unroll
          for (int j = 0; j < 8; ++j)
            o[j] = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(y[j]), 0x128, 0xf, 0xf, false));
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) o[j] = __shfl(y[j], rotated ? partner : lane);
        }
        if (rotated) {
#pragma unroll
          for (int j = 0; j < 8; ++j) y[j] = rope_rotate(y[j], o[j], f[j], first);
        }
        st16((which ? ko + row * ko_row + head * ko_head : qo + row * qo_row + head * qo_head) + 8 * c, pack8(y));
      }
    }
    b ^= 1;
  }
}

// out[s][h*D + d] = bf16(O[s][h][d] * g[s][h])
template <int D>
__global__ __launch_bounds__(256) void head_gate_kernel(const uint16_t *__restrict__ o, int64_t o_row,
                                                        int64_t o_head, const uint16_t *__restrict__ gate,
                                                        int64_t g_row, uint16_t *__restrict__ out, int64_t out_row,
                                                        int64_t n_vec, int heads) {
  constexpr int LANES = D / 8;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t vec = t / LANES;
  const int c = (int)(t % LANES);
  if (vec >= n_vec) return;
  const int head = (int)(vec % heads);
  const int64_t row = vec / heads;
  float x[8], y[8];
  unpack8(ld16(o + row * o_row + head * o_head + 8 * c), x);
  const float g = bf2f(gate[row * g_row + head]);
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = x[j] * g;
  st16(out + row * out_row + (int64_t)head * D + 8 * c, pack8(y));
}

int check_rows(const void *p, int64_t row, int64_t head, const char *name) {
  VDNH3_HOST_CHECK(p != nullptr, VDNH3_ERR_INVALID, "%s is null", name);
  VDNH3_HOST_CHECK(row % 8 == 0 && head % 8 == 0 && reinterpret_cast<uintptr_t>(p) % 16 == 0, VDNH3_ERR_INVALID,
                   "%s must be 16-byte aligned with row and head strides that are multiples of 8 elements", name);
  return VDNH3_OK;
}

}  // namespace
}  // namespace vdnh3

namespace vdnh3 {
namespace {
int qk_norm(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *k, int64_t k_row, int64_t k_head,
            const uint16_t *q_weight, const uint16_t *k_weight, float q_eps, float k_eps, const float *freqs,
            int64_t f_row,
            int rot, uint16_t *q_out, int64_t qo_row, int64_t qo_head, uint16_t *k_out, int64_t ko_row,
            int64_t ko_head, int seq, int heads, int head_dim, void *stream) {
  VDNH3_HOST_CHECK(head_dim == 64 || head_dim == 128, VDNH3_ERR_INVALID,
                   "qk_rmsnorm supports head_dim 64 or 128, got %d", head_dim);
  VDNH3_HOST_CHECK(seq > 0 && heads > 0, VDNH3_ERR_INVALID, "qk_rmsnorm: seq and heads must be positive");
  int rc = check_rows(q, q_row, q_head, "q");
  if (!rc) rc = check_rows(k, k_row, k_head, "k");
  if (!rc) rc = check_rows(q_out, qo_row, qo_head, "q_out");
  if (!rc) rc = check_rows(k_out, ko_row, ko_head, "k_out");
  if (!rc) rc = check_rows(q_weight, 0, 0, "q_weight");
  if (!rc) rc = check_rows(k_weight, 0, 0, "k_weight");
  if (rc) return rc;
  if (freqs) {
    VDNH3_HOST_CHECK(rot > 0 && rot % 16 == 0 && rot <= head_dim, VDNH3_ERR_INVALID,
                     "rope: rot_dim must be a positive multiple of 16 and at most head_dim %d, got %d", head_dim,
                     rot);
    VDNH3_HOST_CHECK(f_row >= 0 && f_row % 4 == 0 && reinterpret_cast<uintptr_t>(freqs) % 16 == 0,
                     VDNH3_ERR_INVALID, "rope: frequencies must be 16-byte aligned with a row stride multiple of 4");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (freqs) {
    // 4096 workgroups (16 per CU over the launch), each walking ~seq / 4096 rows: at the 40 688 x 40 x 128
    // shape 0.35 ms, 0.61 of HBM peak, against 0.36 ms with 1024 or 2048 and 0.46 ms for one workgroup per
    // 16 vectors (the table re-read per workgroup, one load in flight per thread); RB = 4 passes in flight
    // (84 VGPRs): 2 and 3 are slower, 8 takes 246 VGPRs and halves the occupancy (0.67 ms)
    const dim3 grid((unsigned)(seq < 4096 ? seq : 4096));
    if (head_dim == 128)
      hipLaunchKernelGGL((qk_rmsnorm_rope_kernel<128>), grid, dim3(256), 0, s, q, q_row, q_head, k, k_row,
                         k_head, q_weight, k_weight, q_eps, k_eps, freqs, f_row, rot, q_out, qo_row, qo_head, k_out,
                         ko_row, ko_head, seq, heads);
    else
      hipLaunchKernelGGL((qk_rmsnorm_rope_kernel<64>), grid, dim3(256), 0, s, q, q_row, q_head, k, k_row,
                         k_head, q_weight, k_weight, q_eps, k_eps, freqs, f_row, rot, q_out, qo_row, qo_head, k_out,
                         ko_row, ko_head, seq, heads);
    return check_launch("qk_rmsnorm_rope");
  }
  const int64_t n_vec = (int64_t)seq * 2 * heads;
  const dim3 grid((unsigned)((n_vec * (head_dim / 8) + 255) / 256));
  if (head_dim == 128)
    hipLaunchKernelGGL(qk_rmsnorm_kernel<128>, grid, dim3(256), 0, s, q, q_row, q_head, k, k_row, k_head, q_weight,
                       k_weight, q_eps, k_eps, q_out, qo_row, qo_head, k_out, ko_row, ko_head, n_vec, heads);
  else
    hipLaunchKernelGGL(qk_rmsnorm_kernel<64>, grid, dim3(256), 0, s, q, q_row, q_head, k, k_row, k_head, q_weight,
                       k_weight, q_eps, k_eps, q_out, qo_row, qo_head, k_out, ko_row, ko_head, n_vec, heads);
  return check_launch("qk_rmsnorm");
}
}  // namespace
}  // namespace vdnh3

extern "C" int vdnh3_qk_rmsnorm(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *k, int64_t k_row,
                                int64_t k_head, const uint16_t *q_weight, const uint16_t *k_weight, float q_eps,
                                float k_eps, uint16_t *q_out, int64_t qo_row, int64_t qo_head, uint16_t *k_out, int64_t ko_row,
                                int64_t ko_head, int seq, int heads, int head_dim, void *stream) {
  return vdnh3::qk_norm(q, q_row, q_head, k, k_row, k_head, q_weight, k_weight, q_eps, k_eps, nullptr, 0, 0, q_out,
                        qo_row,
                        qo_head, k_out, ko_row, ko_head, seq, heads, head_dim, stream);
}

extern "C" int vdnh3_qk_rmsnorm_rope(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *k,
                                     int64_t k_row, int64_t k_head, const uint16_t *q_weight,
                                     const uint16_t *k_weight, float eps, const float *freqs, int64_t freqs_row,
                                     int rot_dim, uint16_t *q_out, int64_t qo_row, int64_t qo_head, uint16_t *k_out,
                                     int64_t ko_row, int64_t ko_head, int seq, int heads, int head_dim,
                                     void *stream) {
  VDNH3_HOST_CHECK(freqs != nullptr, VDNH3_ERR_INVALID, "rope: null frequencies");
  return vdnh3::qk_norm(q, q_row, q_head, k, k_row, k_head, q_weight, k_weight, eps, eps, freqs, freqs_row, rot_dim,
                        q_out, qo_row, qo_head, k_out, ko_row, ko_head, seq, heads, head_dim, stream);
}

extern "C" int vdnh3_head_gate(const uint16_t *o, int64_t o_row, int64_t o_head, const uint16_t *gate, int64_t gate_row,
                               uint16_t *out, int64_t out_row, int seq, int heads, int head_dim, void *stream) {
  using namespace vdnh3;
  VDNH3_HOST_CHECK(head_dim == 64 || head_dim == 128, VDNH3_ERR_INVALID,
                   "head_gate supports head_dim 64 or 128, got %d", head_dim);
  VDNH3_HOST_CHECK(seq > 0 && heads > 0 && gate != nullptr, VDNH3_ERR_INVALID, "head_gate: empty or null operand");
  int rc = check_rows(o, o_row, o_head, "o");
  if (!rc) rc = check_rows(out, out_row, head_dim, "out");
  if (rc) return rc;
  const int64_t n_vec = (int64_t)seq * heads;
  const int64_t threads = n_vec * (head_dim / 8);
  const dim3 grid((unsigned)((threads + 255) / 256));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (head_dim == 128)
    hipLaunchKernelGGL(head_gate_kernel<128>, grid, dim3(256), 0, s, o, o_row, o_head, gate, gate_row, out, out_row,
                       n_vec, heads);
  else
    hipLaunchKernelGGL(head_gate_kernel<64>, grid, dim3(256), 0, s, o, o_row, o_head, gate, gate_row, out, out_row,
                       n_vec, heads);
  return check_launch("head_gate");
}
