// Block-sparse local-window softmax attention for gfx950 (MI355X), bf16 MFMA.
//
// Computes O_i = softmax(scale * q_i K_A(i)^T) V_A(i) for the VDN-H3 window mask
// (vdn_h3/window.py:331-342) from a host-built tile plan (window_plan.cpp), with an
// optional fused per-head sigmoid gate (vdn_h3/hybrid.py:518-529).
//
// Work decomposition
//   one workgroup = 4 wavefronts = 128 query rows of one head x the key tiles of its run;
//   each wavefront owns 32 query rows and keeps its Q fragment in registers.
//   Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16: every lane
//   then owns one query column (lane % 32) and 16+16 of the 64 keys of a tile, so the row
//   max is one cross-lane exchange (lane ^ 32) and the probabilities P^T feed the next
//   MFMA (O^T += V^T P^T) straight from registers, without an LDS round trip.
//   V^T is read from a head-major copy made by a pre-pass (one extra 2*S*H*D-byte sweep),
//   stored with keys interleaved in 16-key groups so that each lane's 8 MFMA k-values are
//   one 16-byte LDS read.
//
// Scheduling
//   work items (query block, head) are ordered longest-first per head, and the flat
//   workgroup index is remapped so that each XCD (workgroups are dealt round-robin over
//   the 8 XCDs) runs a contiguous slice of that order: the ~64 resident workgroups of an
//   XCD work on the same head and neighbouring query blocks, so their K/V tiles are
//   shared in that XCD's L2.
#include "common.h"

namespace vdnh3 {
namespace {

constexpr int kBM = 128;  // query rows per workgroup
constexpr int kBN = 64;   // keys per tile
constexpr int kThreads = 256;
constexpr float kLazy = 8.0f;  // log2 of the largest probability a stale running max allows

// LDS position p (0..15) inside a 16-key group holds key offset kperm(p): the order in
// which the S^T accumulator of lane group g = p / 8 enumerates its 8 keys of a k-step.
__host__ __device__ constexpr int kperm(int p) { return 8 * ((p & 7) >> 2) + 4 * (p >> 3) + (p & 3); }

// ---------------------------------------------------------------------------------
// Pre-pass: V [seq, heads, D] (strided view) -> vt[head][d][s_pad], keys in kperm order
// inside each 16-key group, zero beyond seq.
// grid (s_pad / 64, heads), 256 threads.
template <int D>
__global__ __launch_bounds__(kThreads) void vt_prepass_kernel(const uint16_t *__restrict__ v, int64_t v_row,
                                                              int64_t v_head, uint16_t *__restrict__ vt,
                                                              int seq, int s_pad) {
  constexpr int P = D + 8;
  __shared__ __attribute__((aligned(16))) uint16_t tile[64 * P];
  const int k0 = blockIdx.x * 64, head = blockIdx.y, tid = threadIdx.x;
  constexpr int CH = D / 8;  // 16-byte chunks per key row
  for (int c = tid; c < 64 * CH; c += kThreads) {
    int r = c / CH, col = c % CH, key = k0 + r;
    uint4 val = make_uint4(0, 0, 0, 0);
    if (key < seq) val = *reinterpret_cast<const uint4 *>(v + key * v_row + head * v_head + col * 8);
    *reinterpret_cast<uint4 *>(&tile[r * P + col * 8]) = val;
  }
  __syncthreads();
  uint16_t *dst = vt + (int64_t)head * D * s_pad + k0;
  for (int c = tid; c < D * 8; c += kThreads) {
    int d = c >> 3, pc = c & 7;  // output positions 8*pc .. 8*pc+7 of row d
    uint16_t e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      int p = 8 * pc + j;
      e[j] = tile[((p & ~15) + kperm(p & 15)) * P + d];
    }
    uint4 o;
    o.x = uint32_t(e[0]) | (uint32_t(e[1]) << 16);
    o.y = uint32_t(e[2]) | (uint32_t(e[3]) << 16);
    o.z = uint32_t(e[4]) | (uint32_t(e[5]) << 16);
    o.w = uint32_t(e[6]) | (uint32_t(e[7]) << 16);
    *reinterpret_cast<uint4 *>(dst + (int64_t)d * s_pad + 8 * pc) = o;
  }
}

// ---------------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(kThreads, 2) void window_attn_kernel(
    const uint16_t *__restrict__ q, int64_t q_row, int64_t q_head, const uint16_t *__restrict__ k, int64_t k_row,
    int64_t k_head, const uint16_t *__restrict__ vt, int s_pad, uint16_t *__restrict__ out, int64_t o_row,
    int64_t o_head, const uint16_t *__restrict__ gate, int64_t g_row, int seq, float scale_log2,
    const int4 *__restrict__ items, int n_items, const int2 *__restrict__ tiles, int per_xcd, int total) {
  constexpr int KP = D + 8;    // K tile row pitch (elements): 16-byte pad -> conflict-free 16-row reads
  constexpr int VP = kBN + 8;  // V^T tile row pitch
  constexpr int NS = D / 16;   // k-steps of the QK^T contraction
  constexpr int NO = D / 32;   // 32-row blocks of O^T
  constexpr int KCH = kBN * D / 8 / kThreads;  // 16-byte K chunks per thread
  constexpr int VCH = D * kBN / 8 / kThreads;  // 16-byte V^T chunks per thread
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kBN * KP];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[D * VP];

  const int bid = blockIdx.x;
  const int L = (bid & 7) * per_xcd + (bid >> 3);
  if (L >= total) return;
  const int head = L / n_items;
  const int4 item = items[L - head * n_items];
  const int q0 = item.x, q1 = item.y, toff = item.z, tcnt = item.w;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int qr = q0 + wave * 32 + l32;
  const int qrc = min(qr, q1 - 1);

  bf16x8_t qf[NS];
  {
    const uint16_t *qp = q + (int64_t)qrc * q_row + (int64_t)head * q_head + 8 * g;
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[s] = as_bf16x8(ld16(qp + 16 * s));
  }

  f32x16_t oacc[NO];
#pragma unroll
  for (int m = 0; m < NO; ++m) oacc[m] = f32x16_t{};
  float m_run = -INFINITY, l_run = 0.f;

  const uint16_t *kbase = k + (int64_t)head * k_head;
  const uint16_t *vbase = vt + (int64_t)head * D * s_pad;
  // per-thread 16-byte chunk coordinates of the K tile ([kBN][D]) and of the V^T tile ([D][kBN])
  int k_r[KCH], k_c[KCH], v_d[VCH], v_c[VCH];
#pragma unroll
  for (int i = 0; i < KCH; ++i) {
    const int c = tid + kThreads * i;
    k_r[i] = c / (D / 8);
    k_c[i] = c % (D / 8);
  }
#pragma unroll
  for (int i = 0; i < VCH; ++i) {
    const int c = tid + kThreads * i;
    v_d[i] = c >> 3;
    v_c[i] = c & 7;
  }
  u32x4_t kreg[KCH], vreg[VCH];
  {
    const int ks = tiles[toff].x;
#pragma unroll
    for (int i = 0; i < KCH; ++i)
      kreg[i] = ld16(kbase + (int64_t)min(ks + k_r[i], seq - 1) * k_row + k_c[i] * 8);
#pragma unroll
    for (int i = 0; i < VCH; ++i)
      vreg[i] = ld16(vbase + (int64_t)v_d[i] * s_pad + ks + v_c[i] * 8);
  }

  for (int t = 0; t < tcnt; ++t) {
    const int packed = tiles[toff + t].y;
#pragma unroll
    for (int i = 0; i < KCH; ++i) st16(&Ks[k_r[i] * KP + k_c[i] * 8], kreg[i]);
#pragma unroll
    for (int i = 0; i < VCH; ++i) st16(&Vs[v_d[i] * VP + v_c[i] * 8], vreg[i]);
    __syncthreads();
    if (t + 1 < tcnt) {
      const int ks = tiles[toff + t + 1].x;
#pragma unroll
      for (int i = 0; i < KCH; ++i)
        kreg[i] = ld16(kbase + (int64_t)min(ks + k_r[i], seq - 1) * k_row + k_c[i] * 8);
#pragma unroll
      for (int i = 0; i < VCH; ++i)
        vreg[i] = ld16(vbase + (int64_t)v_d[i] * s_pad + ks + v_c[i] * 8);
    }

    // S^T = K Q^T : two 32-key blocks x 32 queries
    f32x16_t sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sacc[kb] = f32x16_t{};
      const uint16_t *kp = &Ks[(32 * kb + l32) * KP + 8 * g];
#pragma unroll
      for (int s = 0; s < NS; ++s)
        sacc[kb] = mfma_bf16_32x32x16(as_bf16x8(ld16(kp + 16 * s)), qf[s], sacc[kb]);
    }
    const int lo = packed & 0xffff, hi = packed >> 16;
    if (lo > 0 || hi < kBN) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int ko = 32 * kb + 8 * (i >> 2) + 4 * g + (i & 3);
          if (ko < lo || ko >= hi) sacc[kb][i] = -INFINITY;
        }
    }
    // Online softmax in base 2, one query per lane. The running max m_run only moves when
    // this tile's max exceeds it by more than 2^kLazy: probabilities are then bounded by
    // 2^kLazy (exact softmax either way, since a common shift cancels in O / l), and most
    // tiles skip rescaling the accumulators.
    float mt = fmaxf(sacc[0][0], sacc[0][1]);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; i += 2) mt = fmaxf(mt, fmaxf(sacc[kb][i], sacc[kb][i + 1]));
    mt = fmaxf(mt, __shfl_xor(mt, 32)) * scale_log2;
    const bool grow = mt > m_run + kLazy;
    if (__any(grow)) {
      const float m_new = grow ? mt : m_run;
      const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= corr;
#pragma unroll
      for (int m = 0; m < NO; ++m) oacc[m] *= corr;
    }
    float rs = 0.f;
    bf16x8_t pb[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p = __builtin_amdgcn_exp2f(fmaf(sacc[kb][i], scale_log2, -m_run));
        rs += p;
        pb[2 * kb + (i >> 3)][i & 7] = (__bf16)p;
      }
    l_run += rs;

    // O^T += V^T P^T : NO blocks of 32 d-rows, 4 k-steps of 16 keys
#pragma unroll
    for (int m = 0; m < NO; ++m) {
      const uint16_t *vp = &Vs[(32 * m + l32) * VP + 8 * g];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
        oacc[m] = mfma_bf16_32x32x16(as_bf16x8(ld16(vp + 16 * tt)), pb[tt], oacc[m]);
    }
    __syncthreads();
  }

  l_run += __shfl_xor(l_run, 32);
  const float inv = 1.f / l_run;
  if (qr < q1) {
    float gv = 1.f;
    if (gate) gv = bf2f(gate[(int64_t)qr * g_row + head]);
    uint16_t *op = out + (int64_t)qr * o_row + (int64_t)head * o_head;
#pragma unroll
    for (int m = 0; m < NO; ++m)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        float v0 = round_bf(oacc[m][4 * i4 + 0] * inv), v1 = round_bf(oacc[m][4 * i4 + 1] * inv);
        float v2 = round_bf(oacc[m][4 * i4 + 2] * inv), v3 = round_bf(oacc[m][4 * i4 + 3] * inv);
        if (gate) {
          v0 *= gv;
          v1 *= gv;
          v2 *= gv;
          v3 *= gv;
        }
        uint2 w;
        w.x = pack_bf2(v0, v1);
        w.y = pack_bf2(v2, v3);
        *reinterpret_cast<uint2 *>(op + 32 * m + 8 * i4 + 4 * g) = w;
      }
  }
}

template <int D>
int launch_prepass(const uint16_t *v, int64_t v_row, int64_t v_head, int seq, int heads, void *workspace,
                   hipStream_t stream) {
  const int s_pad = (seq + 63) / 64 * 64;
  hipLaunchKernelGGL(vt_prepass_kernel<D>, dim3(s_pad / 64, heads), dim3(kThreads), 0, stream, v, v_row, v_head,
                     static_cast<uint16_t *>(workspace), seq, s_pad);
  return check_launch("window vt_prepass");
}

template <int D>
int launch_attn(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *k, int64_t k_row, int64_t k_head,
                uint16_t *out, int64_t o_row, int64_t o_head, const uint16_t *gate, int64_t gate_row, int seq,
                int heads, float scale, const int32_t *items, int32_t n_items, const int32_t *tiles,
                const void *workspace, hipStream_t stream) {
  const int s_pad = (seq + 63) / 64 * 64;
  const int total = n_items * heads;
  const int per_xcd = (total + 7) / 8;
  hipLaunchKernelGGL(window_attn_kernel<D>, dim3(per_xcd * 8), dim3(kThreads), 0, stream, q, q_row, q_head, k,
                     k_row, k_head, static_cast<const uint16_t *>(workspace), s_pad, out, o_row, o_head, gate,
                     gate_row, seq, scale * 1.4426950408889634f, reinterpret_cast<const int4 *>(items), n_items,
                     reinterpret_cast<const int2 *>(tiles), per_xcd, total);
  return check_launch("window_attn");
}

int check_common(int seq, int heads, int head_dim, const void *workspace, size_t workspace_bytes) {
  VDNH3_HOST_CHECK(head_dim == 64 || head_dim == 128, VDNH3_ERR_INVALID,
                   "window attention supports head_dim 64 or 128, got %d", head_dim);
  VDNH3_HOST_CHECK(seq > 0 && heads > 0, VDNH3_ERR_INVALID, "seq and heads must be positive");
  VDNH3_HOST_CHECK(workspace != nullptr, VDNH3_ERR_INVALID, "null workspace");
  VDNH3_HOST_CHECK(workspace_bytes >= vdnh3_window_workspace_bytes(seq, heads, head_dim), VDNH3_ERR_INVALID,
                   "workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
                   vdnh3_window_workspace_bytes(seq, heads, head_dim));
  return VDNH3_OK;
}

int check_vec(const void *p, int64_t row, int64_t head, const char *name) {
  VDNH3_HOST_CHECK(p != nullptr, VDNH3_ERR_INVALID, "%s is null", name);
  VDNH3_HOST_CHECK(row % 8 == 0 && head % 8 == 0 && reinterpret_cast<uintptr_t>(p) % 16 == 0, VDNH3_ERR_INVALID,
                   "%s must be 16-byte aligned with row and head strides that are multiples of 8 elements", name);
  return VDNH3_OK;
}

}  // namespace
}  // namespace vdnh3

extern "C" int vdnh3_window_block_m(void) { return vdnh3::kBM; }
extern "C" int vdnh3_window_block_n(void) { return vdnh3::kBN; }

extern "C" size_t vdnh3_window_workspace_bytes(int seq, int heads, int head_dim) {
  if (seq <= 0 || heads <= 0 || head_dim <= 0) return 0;
  return size_t(heads) * size_t(head_dim) * size_t((seq + 63) / 64 * 64) * sizeof(uint16_t);
}

extern "C" int vdnh3_window_vt_prepass(const uint16_t *v, int64_t v_row, int64_t v_head, int seq, int heads,
                                       int head_dim, void *workspace, size_t workspace_bytes, void *stream) {
  int rc = vdnh3::check_common(seq, heads, head_dim, workspace, workspace_bytes);
  if (!rc) rc = vdnh3::check_vec(v, v_row, v_head, "v");
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return head_dim == 128 ? vdnh3::launch_prepass<128>(v, v_row, v_head, seq, heads, workspace, s)
                         : vdnh3::launch_prepass<64>(v, v_row, v_head, seq, heads, workspace, s);
}

extern "C" int vdnh3_window_attn_prepared(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *k,
                                          int64_t k_row, int64_t k_head, uint16_t *out, int64_t o_row,
                                          int64_t o_head, const uint16_t *gate, int64_t gate_row, int seq, int heads,
                                          int head_dim, float scale, const int32_t *items, int32_t n_items,
                                          const int32_t *tiles, const void *workspace, size_t workspace_bytes,
                                          void *stream) {
  int rc = vdnh3::check_common(seq, heads, head_dim, workspace, workspace_bytes);
  if (!rc) rc = vdnh3::check_vec(q, q_row, q_head, "q");
  if (!rc) rc = vdnh3::check_vec(k, k_row, k_head, "k");
  if (rc) return rc;
  VDNH3_HOST_CHECK(out != nullptr && o_row % 4 == 0 && o_head % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 8 == 0,
                   VDNH3_ERR_INVALID, "out must be 8-byte aligned with strides that are multiples of 4 elements");
  VDNH3_HOST_CHECK(items != nullptr && tiles != nullptr && n_items > 0, VDNH3_ERR_INVALID, "empty window plan");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (head_dim == 128)
    return vdnh3::launch_attn<128>(q, q_row, q_head, k, k_row, k_head, out, o_row, o_head, gate, gate_row, seq, heads,
                                   scale, items, n_items, tiles, workspace, s);
  return vdnh3::launch_attn<64>(q, q_row, q_head, k, k_row, k_head, out, o_row, o_head, gate, gate_row, seq, heads,
                                scale, items, n_items, tiles, workspace, s);
}

extern "C" int vdnh3_window_attn_fwd(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *k,
                                     int64_t k_row, int64_t k_head, const uint16_t *v, int64_t v_row, int64_t v_head,
                                     uint16_t *out, int64_t o_row, int64_t o_head, const uint16_t *gate,
                                     int64_t gate_row, int seq, int heads, int head_dim, float scale,
                                     const int32_t *items, int32_t n_items, const int32_t *tiles, void *workspace,
                                     size_t workspace_bytes, void *stream) {
  int rc = vdnh3_window_vt_prepass(v, v_row, v_head, seq, heads, head_dim, workspace, workspace_bytes, stream);
  if (rc) return rc;
  return vdnh3_window_attn_prepared(q, q_row, q_head, k, k_row, k_head, out, o_row, o_head, gate, gate_row, seq,
                                    heads, head_dim, scale, items, n_items, tiles, workspace, workspace_bytes, stream);
}
