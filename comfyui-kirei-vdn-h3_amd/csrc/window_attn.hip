// Block-sparse local-window softmax attention for gfx950 (MI355X), bf16 MFMA.
//
// Computes O_i = softmax(scale * q_i K_A(i)^T) V_A(i) for the VDN-H3 window mask
// (vdn_h3/window.py:331-342) from a host-built tile plan (window_plan.cpp), with an
// optional fused per-head sigmoid gate (vdn_h3/hybrid.py:518-529).
//
// Work decomposition
//   one workgroup = 8 wavefronts = 256 query rows of one head x the key tiles of its run;
//   each wavefront owns 32 query rows and keeps its Q fragment in registers.
//   Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16: every lane
//   then owns one query column (lane % 32) and 3 x 16 of the 96 keys of a tile, so the row
//   max is one cross-lane exchange (lane ^ 32) and the probabilities P^T feed the next
//   MFMA (O^T += V^T P^T) straight from registers, without an LDS round trip.
//   V^T is read from a copy made by a pre-pass (one extra 2*S*H*D-byte sweep): per head, one
//   contiguous image per 96-key tile, its 16-byte chunks already in the order and XOR swizzle of
//   the kernel's LDS tile, with keys interleaved in 16-key groups so that each lane's 8 MFMA
//   k-values are one 16-byte LDS read. K and V^T tiles go straight from HBM/L2 to LDS rings
//   (global_load_lds_dwordx4), each wavefront's load of a V^T tile one contiguous kilobyte; the
//   two halves of the workgroup alternate between the matrix cores and the VALU (see
//   window_attn_kernel).
//
// Scheduling
//   work items (query block, head) are ordered longest-first per head, and the flat
//   workgroup index is remapped so that each XCD (workgroups are dealt round-robin over
//   the 8 XCDs) runs a contiguous slice of that order: the resident workgroups of an
//   XCD work on the same head and neighbouring query blocks, so their K/V tiles are
//   shared in that XCD's L2.
#include "common.h"
#include "qk_norm.h"

namespace vdnh3 {
namespace {

constexpr int kBM = 256;  // query rows per workgroup (8 wavefronts x 32)
constexpr int kBN = 96;   // keys per tile: 48 MFMAs per wavefront and phase at D = 128
constexpr int kThreads = 512;
constexpr int kRing = 3;  // LDS slots per K and V^T ring (144 KB at D = 128): loads run kRing - 1 tiles ahead
constexpr float kLazy = 8.0f;  // log2 of the largest probability a stale running max allows

// LDS position p (0..15) inside a 16-key group holds key offset kperm(p): the order in
// which the S^T accumulator of lane group g = p / 8 enumerates its 8 keys of a k-step.
__host__ __device__ constexpr int kperm(int p) { return 8 * ((p & 7) >> 2) + 4 * (p >> 3) + (p & 3); }

// ---------------------------------------------------------------------------------
// LDS slots of the staged tiles. Each tile row is split into 16-byte chunks; chunk c of row r
// is stored at slot c ^ swizzle(r), so that the 16 lanes of one MFMA fragment read (16
// consecutive rows, one chunk column) hit 16 different 16-byte bank groups.
template <int D>
__device__ __forceinline__ int k_slot(int r, int c) {
  if constexpr (D == 128) return c ^ (r & 15);  // 16 chunks per 256-byte row
  else return c ^ ((r >> 1) & 7);               // 8 chunks per 128-byte row
}
__device__ __forceinline__ int v_slot(int d, int c) { return c ^ ((d >> 1) & 7); }  // 8 chunks per row
// the V^T tile's 32-key part (4 chunks per row): the 16 lanes of a fragment read (rows d..d+15)
// hit 16 different 16-byte bank groups
__device__ __forceinline__ int vb_slot(int d, int c) { return c ^ ((d >> 2) & 3); }

// Rows of the V^T copy and of the normalised q / k regions: seq rounded up to 192, a multiple of the
// pre-passes' 64-row blocks and of the attention's 96-key tiles, so a tile never reads past its head's
// region.
__host__ __device__ constexpr int pad_rows(int seq) { return (seq + 191) / 192 * 192; }

// ---------------------------------------------------------------------------------
// The V^T copy is a sequence of tile images, one per 96-key tile: the image of keys [ks, ks + 96)
// of head h starts at element (h * s_pad + ks) * D and holds the tile's 16-byte chunks in LDS
// order: position P < 8 D is (d = P / 8, slot P % 8) of the 64-key part, holding chunk
// v_slot(d, slot) of keys [ks, ks + 64) of V^T row d; position 8 D + 4 d + slot of the 32-key part
// holds chunk vb_slot(d, slot) of keys [ks + 64, ks + 96). Inside a chunk the 8 keys follow kperm
// within their 16-key group; keys past seq are zero. A tile load is then a contiguous copy.
// write_vt_image: the image chunks of the 64 keys [k0, k0 + 64) (k0 a multiple of 64) from their V rows
// staged in LDS (row r at rows + r * P), into the head's images at vt_head. A 64-key block holds whole
// 16-key groups, so every chunk it writes is complete; it covers one or two tiles.
template <int D, int P>
__device__ __forceinline__ void write_vt_image(const uint16_t *rows, int k0, uint16_t *__restrict__ vt_head,
                                               int tid) {
  for (int cc = tid; cc < D * 8; cc += kThreads) {
    const int d = cc >> 3, pc = cc & 7;  // V^T row; chunk pc holds key slots 8 pc .. 8 pc + 7 of the block
    const int key = k0 + 8 * pc, tile = key / kBN, sb = key - tile * kBN;
    const int pos = sb < 64 ? 8 * d + v_slot(d, sb >> 3) : 8 * D + 4 * d + vb_slot(d, (sb - 64) >> 3);
    uint16_t e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int p = 8 * pc + j;
      e[j] = rows[((p & ~15) + kperm(p & 15)) * P + d];
    }
    uint4 o;
    o.x = uint32_t(e[0]) | (uint32_t(e[1]) << 16);
    o.y = uint32_t(e[2]) | (uint32_t(e[3]) << 16);
    o.z = uint32_t(e[4]) | (uint32_t(e[5]) << 16);
    o.w = uint32_t(e[6]) | (uint32_t(e[7]) << 16);
    *reinterpret_cast<uint4 *>(vt_head + (int64_t)tile * (kBN * D) + pos * 8) = o;
  }
}

// ---------------------------------------------------------------------------------
// Pre-pass: V [seq, heads, D] (strided view) -> the V^T tile images, 64 keys per workgroup.
// grid (s_pad / 64, heads), kThreads threads.
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
  write_vt_image<D, P>(tile, k0, vt + (int64_t)head * s_pad * D, tid);
}

// ---------------------------------------------------------------------------------
// The block's q_norm / k_norm (RMSNorm over the head dim, with ROPE the split-half rotation, one
// bf16 rounding: the arithmetic of qk_norm.h) of the BR rows [k0, k0 + BR) of one head at a
// time, written head-major (row r at dst + r * D), zero for rows at or past seq. Each row is
// normalised by an aligned group of D/8 lanes, one 8-channel chunk per lane (THREADS / (D/8) rows
// per pass; with D = 64 the last pass is partly idle). A lane loads the RoPE matrix rows its chunk
// uses once (the constructor) and reuses them for every head (run): row 0 (f00, f01) below half,
// row 1 (f10, f11) above.
template <int D, bool ROPE, int THREADS, int BR>
struct RowNorm {
  static constexpr int CH = D / 8, ROWS = THREADS / CH, ITER = (BR + ROWS - 1) / ROWS;
  // row r0 + it * ROWS lies in the block (a whole row group is in or out)
  __device__ __forceinline__ bool in_block(int it) const { return BR % ROWS == 0 || r0 + it * ROWS < BR; }
  int c, r0, half, k0, seq;
  bool first, rotated;
  float2 fm[ITER][ROPE ? 8 : 1];

  __device__ __forceinline__ RowNorm(const float *__restrict__ freqs, int64_t f_row, int rot, int k0_, int seq_,
                                     int tid)
      : c(tid % CH), r0(tid / CH), half(rot >> 1), k0(k0_), seq(seq_) {
    first = 8 * c < half;
    rotated = ROPE && 8 * c < rot;
    if constexpr (ROPE) {
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int key = k0 + r0 + it * ROWS;
        if (rotated && key < seq && in_block(it)) {
          const float *f = freqs + key * f_row + 4 * (first ? 8 * c : 8 * c - half) + (first ? 0 : 2);
#pragma unroll
          for (int j = 0; j < 8; ++j) fm[it][j] = *reinterpret_cast<const float2 *>(f + 4 * j);
        }
      }
    }
  }

  __device__ __forceinline__ void run(const uint16_t *__restrict__ x, int64_t x_row, int64_t x_head,
                                      const uint16_t *__restrict__ weight, float eps, uint16_t *__restrict__ dst,
                                      int head) const {
    float wf[8];
    {
      const u32x4_t w = ld16(weight + 8 * c);
#pragma unroll
      for (int j = 0; j < 8; ++j) wf[j] = __uint_as_float((j & 1) ? (w[j >> 1] & 0xffff0000u) : (w[j >> 1] << 16));
    }
    u32x4_t raw[ITER];
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
      const int key = k0 + r0 + it * ROWS;
      raw[it] = key < seq && in_block(it) ? ld16(x + key * x_row + head * x_head + 8 * c) : u32x4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
      if (!in_block(it)) continue;
      const int r = r0 + it * ROWS;
      const bool live = k0 + r < seq;
      float xf[8], y[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        xf[j] = __uint_as_float((j & 1) ? (raw[it][j >> 1] & 0xffff0000u) : (raw[it][j >> 1] << 16));
      const float rr = rms_factor(group_tree_sum<CH>(chunk_sumsq(xf)), D, eps);
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = xf[j] * rr * wf[j];
      if constexpr (ROPE) {
        // the partner chunk (8c +- half) is lane c +- half / 8 of the same row group
        const int lane = __lane_id(), step = half >> 3;
        const int partner = rotated ? (first ? lane + step : lane - step) : lane;
        float o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = __shfl(y[j], partner);
        if (rotated && live) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float2 m = fm[it][j];
            y[j] = rope_rotate(y[j], o[j], f32x4_t{m.x, m.y, m.x, m.y}, first);
          }
        }
      }
      if (!live) {
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = 0.f;
      }
      st16(dst + r * D + 8 * c, u32x4_t{pack_bf2(y[0], y[1]), pack_bf2(y[2], y[3]), pack_bf2(y[4], y[5]),
                                        pack_bf2(y[6], y[7])});
    }
  }
};

constexpr int kPrepassHeads = 10;  // heads per pre-pass workgroup (they share its rows' RoPE matrices);
                                   // 10 measured 4% faster than 8 at 40 heads, 4, 5 and 20 no better

// Pre-pass of the normalising attention, for the 64 rows [k0, k0 + 64) of up to kPrepassHeads
// heads: the V^T image chunks of vt_prepass_kernel, the normalised keys kn[head][key][d] and, when q
// is given, the normalised queries qn[head][row][d] (RowNorm). V tiles alternate between two LDS
// buffers, so one barrier per head orders the tile's writes before its transposed reads, and the
// reads of a buffer before its next writes.
template <int D, bool ROPE>
__global__ __launch_bounds__(kThreads) void qkv_prepass_kernel(
    const uint16_t *__restrict__ q, int64_t q_row, int64_t q_head, const uint16_t *__restrict__ q_weight, float q_eps,
    const uint16_t *__restrict__ k, int64_t k_row, int64_t k_head, const uint16_t *__restrict__ k_weight, float k_eps,
    const uint16_t *__restrict__ v, int64_t v_row, int64_t v_head, const float *__restrict__ freqs, int64_t f_row,
    int rot, uint16_t *__restrict__ vt, uint16_t *__restrict__ kn, uint16_t *__restrict__ qn, int seq, int s_pad,
    int heads) {
  constexpr int P = D + 8;
  constexpr int CH = D / 8;  // 16-byte chunks per row
  __shared__ __attribute__((aligned(16))) uint16_t tile[2][64 * P];
  const int h0 = blockIdx.x * kPrepassHeads, h1 = min(heads, h0 + kPrepassHeads);
  const int k0 = blockIdx.y * 64, tid = threadIdx.x;
  const RowNorm<D, ROPE, kThreads, 64> norm(freqs, f_row, rot, k0, seq, tid);
  for (int head = h0; head < h1; ++head) {
    uint16_t *buf = tile[head & 1];
    for (int cc = tid; cc < 64 * CH; cc += kThreads) {
      int r = cc / CH, col = cc % CH, key = k0 + r;
      uint4 val = make_uint4(0, 0, 0, 0);
      if (key < seq) val = *reinterpret_cast<const uint4 *>(v + key * v_row + head * v_head + col * 8);
      *reinterpret_cast<uint4 *>(&buf[r * P + col * 8]) = val;
    }
    const int64_t off = ((int64_t)head * s_pad + k0) * D;
    norm.run(k, k_row, k_head, k_weight, k_eps, kn + off, head);
    if (q) norm.run(q, q_row, q_head, q_weight, q_eps, qn + off, head);
    __syncthreads();
    write_vt_image<D, P>(buf, k0, vt + (int64_t)head * s_pad * D, tid);
  }
}



// The value of lane (l + 32) mod 64, via v_permlane32_swap (gfx950).
__device__ __forceinline__ float other_half(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const uint32_t lane = __lane_id();
  return __uint_as_float(lane < 32 ? r[1] : r[0]);
}

// The Q^T fragments of a wavefront: lane (l32, g) holds channels 16 s + 8 g + j (j < 8) of its
// query row qrc, chunk 2 s + g. QNORM: q is normalised as it is loaded (the block's q_norm with
// q_weight / q_eps, the arithmetic of qk_norm.h); otherwise q is used as given.
template <int D, bool QNORM>
__device__ __forceinline__ void load_q_frags(const uint16_t *__restrict__ q, int64_t q_row, int64_t q_head, int qrc,
                                             int head, int g, const uint16_t *__restrict__ q_weight, float q_eps,
                                             bf16x8_t (&qf)[D / 16]) {
  constexpr int NS = D / 16;
  const uint16_t *qp = q + (int64_t)qrc * q_row + (int64_t)head * q_head + 8 * g;
  if constexpr (!QNORM) {
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[s] = as_bf16x8(ld16(qp + 16 * s));
  } else {
    float y[NS][8], p[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const u32x4_t raw = ld16(qp + 16 * s);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        y[s][j] = __uint_as_float((j & 1) ? (raw[j >> 1] & 0xffff0000u) : (raw[j >> 1] << 16));
      p[s] = chunk_sumsq(y[s]);
    }
    const float rr = rms_factor(halves_tree_sum<NS>(p), D, q_eps);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const u32x4_t w = ld16(q_weight + 16 * s + 8 * g);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        y[s][j] = y[s][j] * rr * __uint_as_float((j & 1) ? (w[j >> 1] & 0xffff0000u) : (w[j >> 1] << 16));
    }
#pragma unroll
    for (int s = 0; s < NS; ++s)
      qf[s] = as_bf16x8(u32x4_t{pack_bf2(y[s][0], y[s][1]), pack_bf2(y[s][2], y[s][3]), pack_bf2(y[s][4], y[s][5]),
                                pack_bf2(y[s][6], y[s][7])});
  }
}

// The output rows of a wavefront: O = O^T / l (l summed over the two half-waves), rounded to bf16,
// times the row's gate when one is given (the gate fused into the attention epilogue).
template <int D>
__device__ __forceinline__ void store_rows(const f32x16_t (&oacc)[D / 32], float l_run, int qr, int q1,
                                           const uint16_t *__restrict__ gate, int64_t g_row, int head,
                                           uint16_t *__restrict__ out, int64_t o_row, int64_t o_head, int g) {
  constexpr int NO = D / 32;
  l_run += other_half(l_run);
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

// ---------------------------------------------------------------------------------
// Two-group ping-pong over the key tiles t = 0..T-1 of a work item (256 query rows of one head).
// Waves 0-3 (group A) and 4-7 (group B) each own 32 query rows; wave w and w + 4 share a SIMD.
// The item runs in barrier-separated phases p = 0 .. 2T+1; in each phase one group works on the
// matrix cores and the other on the VALU, so the two waves of every SIMD alternate:
//   MFMA phase of tile t :  O^T += V(t-1)^T P(t-1)^T   and   S(t)^T = K(t) Q^T      (48 MFMAs)
//   VALU phase of tile t :  P(t) = exp2(scale S(t) - m), row max / sum, O rescale   (softmax)
// Group A runs tile t's MFMA phase in phase 2t and its VALU phase in 2t+1; group B one phase
// later. K(t) and V(t-1) are read in phases 2t and 2t+1 only; tiles are loaded direct to LDS
// into three-slot rings, two tiles ahead: K tiles by group A and V^T tiles by group B, each at
// the start of the issuing group's VALU phase, so the MFMA stream carries no memory instruction
// and a tile that misses L2 has two tiles' time to land. A tile is 96 keys: every phase switch
// (a barrier, the first fragment reads of the MFMA phase) is shared by 48 MFMAs per wavefront, a
// third fewer switches than with 64-key tiles for the same work.
// QNORM: q is normalised as it is loaded (the block's q_norm with q_weight / q_eps, the arithmetic
// of qk_norm.h); otherwise q is used as given.
template <int D, bool QNORM>
__global__ __launch_bounds__(kThreads, 1) void window_attn_kernel(
    const uint16_t *__restrict__ q, int64_t q_row, int64_t q_head, const uint16_t *__restrict__ k, int64_t k_row,
    int64_t k_head, const uint16_t *__restrict__ vt, int s_pad, uint16_t *__restrict__ out, int64_t o_row,
    int64_t o_head, const uint16_t *__restrict__ gate, int64_t g_row, int seq, float scale_log2,
    const int4 *__restrict__ items, int n_items, const int2 *__restrict__ tiles, int per_xcd, int total,
    const uint16_t *__restrict__ q_weight, float q_eps) {
  constexpr int KC = D / 8;    // 16-byte chunks per K row
  constexpr int NS = D / 16;   // k-steps of the QK^T contraction
  constexpr int NO = D / 32;   // 32-row blocks of O^T
  constexpr int NKB = kBN / 32;  // 32-key blocks of S^T
  constexpr int NT = kBN / 16;   // k-steps of the PV contraction
  constexpr int KT = kBN * D, VT = D * kBN;  // elements per tile
  // a V^T tile in LDS: keys 0..63 as [D][8 chunks] (v_slot), then keys 64..95 as [D][4 chunks] (vb_slot)
  constexpr int VA = D * 64;
  static_assert(kBN == 96, "the V^T tile layout is a 64-key part and a 32-key part");
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kRing][KT];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[kRing][VT];

  const int bid = blockIdx.x;
  const int L = (bid & 7) * per_xcd + (bid >> 3);
  if (L >= total) return;
  const int head = L / n_items;
  const int4 item = items[L - head * n_items];
  const int q0 = item.x, q1 = item.y, toff = item.z, T = item.w;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int group = wave >> 2;
  const int qr = q0 + wave * 32 + l32;
  const int qrc = min(qr, q1 - 1);
  // a wavefront whose 32 rows all lie past the item's end (the short last item of a run) skips
  // its fragment reads, MFMAs and softmax; it still issues its share of the tile loads and
  // joins every barrier
  const bool rows_live = q0 + wave * 32 < q1;

  bf16x8_t qf[NS];
  load_q_frags<D, QNORM>(q, q_row, q_head, qrc, head, g, q_weight, q_eps, qf);

  const uint16_t *kbase = k + (int64_t)head * k_head;
  const uint16_t *vbase = vt + (int64_t)head * D * s_pad;
  // Tile loads, by one group of 256 threads: thread chunk i fills LDS position P = 256 i + gtid
  // (16-byte units) of the tile. In a K tile, P is (row P / KC, slot P % KC) and holds chunk
  // slot ^ swizzle(row) of that key row; row kr0 + i * 256 / KC has the same swizzle for every i.
  // A V^T tile image is already in LDS order: P comes from position P of the image.
  // Rows past seq read row seq - 1 (their scores are masked).
  constexpr int KCG = kBN * KC / 256, VCG = D * (kBN / 8) / 256;  // 16-byte chunks per thread and tile
  static_assert(KCG >= 1 && VCG >= 1 && KCG == VCG, "both groups issue the same number of loads");
  const int gtid = tid & 255, gw = wave & 3;
  const int kr0 = gtid / KC;
  const int kslot = k_slot<D>(kr0, gtid % KC) * 8;
  // per-lane byte offsets of this group's chunks inside a tile's source rows (K rows for group
  // A, V^T rows for group B) and the tile's LDS base of this wavefront: an issue is a scalar
  // tile base, a scalar M0 and the load
  uint32_t doff[KCG];
#pragma unroll
  for (int i = 0; i < KCG; ++i) {
    const int P = 256 * i + gtid;
    doff[i] = 2u * (group == 0 ? (uint32_t)((kr0 + i * (256 / KC)) * (int)k_row + kslot) : (uint32_t)(P * 8));
  }
  const uint32_t lds_dma = __builtin_amdgcn_readfirstlane(
      (group == 0 ? lds_address(&Ks[0][0]) : lds_address(&Vs[0][0])) + gw * 64 * 16);
  constexpr uint32_t kTileBytes = KT * 2;
  static_assert(KT == VT, "K and V^T tiles have the same size");
  // this group's loads of the tile whose first key is ks into ring slot `slot`; the last K tile
  // of the sequence reads rows past seq as row seq - 1 (their scores are masked)
  auto tile_dma = [&](int ks, int slot) __device__ {
    const uint16_t *base = group == 0 ? kbase + (int64_t)ks * k_row : vbase + (int64_t)ks * D;
    uint32_t off[KCG];
#pragma unroll
    for (int i = 0; i < KCG; ++i) off[i] = doff[i];
    if (group == 0 && ks + kBN > seq) {  // uniform: taken for the last tile of the sequence only
#pragma unroll
      for (int i = 0; i < KCG; ++i)
        off[i] = 2u * (uint32_t)((min(ks + kr0 + i * (256 / KC), seq - 1) - ks) * (int)k_row + kslot);
    }
#pragma unroll
    for (int i = 0; i < KCG; ++i)
      global_to_lds16_sbase(base, off[i], lds_dma + (uint32_t)slot * kTileBytes + (uint32_t)(i * 256 * 16));
  };

  // Fragment offsets inside a tile (elements). The swizzles depend on the row only through
  // l32 (r = 32 kb + l32, d = 32 m + l32), so the 32-row blocks differ by constant offsets.
  int kfo[NS], vfo[NT];
#pragma unroll
  for (int st = 0; st < NS; ++st) kfo[st] = (l32 * KC + k_slot<D>(l32, 2 * st + g)) * 8;
#pragma unroll
  for (int tt = 0; tt < NT; ++tt)
    vfo[tt] = tt < 4 ? (l32 * 8 + v_slot(l32, 2 * tt + g)) * 8 : VA + (l32 * 4 + vb_slot(l32, 2 * (tt - 4) + g)) * 8;

  f32x16_t oacc[NO], sacc[NKB];
#pragma unroll
  for (int m = 0; m < NO; ++m) oacc[m] = f32x16_t{};
  bf16x8_t pb[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) pb[j] = bf16x8_t{};
  float m_run = -INFINITY, l_run = 0.f;

  // Rings: K(tau) and V(tau) live in slot tau % kRing. K(t) and V(t-1) are read in phases 2t
  // (group A) and 2t+1 (group B). Tile loads are issued by the group in its VALU phase, so the
  // MFMA stream carries no memory instruction: in its VALU phase of tile t, group A issues
  // K(t+kRing-1) (phase 2t+1) over K(t-1), last read in phase 2t-1, and group B issues
  // V(t+kRing-1) (phase 2t+2) over V(t-1), last read in phase 2t+1. In each phase the slot
  // being written differs from the K and V slots the MFMA group reads. Past the end the tile
  // index is clamped to T-1: such loads rewrite
  // slots that no real tile reads any more, and every VALU phase issues the same count, so each
  // group's vmcnt wait at the end of odd phases is exact.
  // prologue: K(0..kRing-2) by group A, V(0..kRing-3) by group B, all landed; V(-1), the V^T
  // slot read by the PV of tile 0 (with P(-1) = 0), is zeroed so that product is exactly zero.
  // Group B's first issue (phase 0) is V(kRing-2).
#pragma unroll
  for (int j = 0; j < kRing - 1; ++j)
    if (j < kRing - 2 || group == 0) tile_dma(tiles[toff + min(j, T - 1)].x, j);
  for (int i = tid; i < VT / 8; i += kThreads) st16(Vs[kRing - 1] + i * 8, u32x4_t{0, 0, 0, 0});
  wait_vm_lds<0>();
  bare_barrier();

  // Descriptors of the next VALU phase of this group (the key start of its tile load and the
  // mask bounds of its tile), scalar loads made at the end of the group's MFMA phase and
  // consumed after the barrier. Group B's first VALU phase (phase 0, tile -1) issues V(kRing-2).
  int dma_ks = group == 0 ? 0 : tiles[toff + min(kRing - 2, T - 1)].x;
  int mask = 0;

  const int phases = 2 * T + 2;
  for (int p = 0; p < phases; ++p) {
    // Group A (B) works on the matrix cores in even (odd) phases. Both tile indices depend on
    // p only, so tile descriptors are scalar loads.
    const int t_mfma = p >> 1;            // A: p = 2t; B: p = 2t + 1
    const int t_valu = (p - 1) >> 1;      // A: p = 2t + 1 (odd); B: p = 2t + 2 (even)
    if (group == (p & 1)) {
      if (!rows_live) {
        // descriptors of this group's next VALU phase (tile t_mfma)
        dma_ks = tiles[toff + min(t_mfma + kRing - 1, T - 1)].x;
      } else {
      // MFMA phase of tile t: O^T += V(t-1)^T P(t-1)^T, S(t)^T = K(t) Q^T (24 + 24 MFMAs at D = 128).
      // t = 0 has no PV and t = T no QK: those phases run on a zero tile / discard the scores,
      // so the phase is one branch-free block. Fragment reads run eight MFMAs ahead.
      const int t = t_mfma;
      const uint16_t *vtile = Vs[(t + kRing - 1) % kRing];
      const uint16_t *ktile = Ks[t % kRing];
      // MFMA i < NP: PV block m = i % NO, k-step tt = i / NO; i >= NP: QK block kb = (i - NP) % NKB,
      // k-step st = (i - NP) / NKB. Consecutive MFMAs update different accumulators, so none waits
      // for the result of the one before it.
      constexpr int NP = NO * NT, NM = NP + NKB * NS;
      auto frag = [&](int i) __device__ {
        if (i < NP) {
          const int m = i % NO, tt = i / NO;
          return ld16(vtile + (tt < 4 ? m * 32 * 64 : m * 32 * 32) + vfo[tt]);
        }
        return ld16(ktile + ((i - NP) % NKB) * 32 * D + kfo[(i - NP) / NKB]);
      };
      // the MFMA wave of each SIMD issues ahead of the VALU wave sharing it
      __builtin_amdgcn_s_setprio(1);
      u32x4_t fr[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) fr[i] = frag(i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < NM; ++i) {
        const u32x4_t a = fr[i & 7];
        if (i < NP) {
          oacc[i % NO] = mfma_bf16_32x32x16(as_bf16x8(a), pb[i / NO], oacc[i % NO]);
        } else {
          const int kb = (i - NP) % NKB, st = (i - NP) / NKB;
          if (st == 0) sacc[kb] = f32x16_t{};
          sacc[kb] = mfma_bf16_32x32x16(as_bf16x8(a), qf[st], sacc[kb]);
        }
        if (i + 8 < NM) fr[i & 7] = frag(i + 8);
        __builtin_amdgcn_sched_barrier(0);
      }
      __builtin_amdgcn_s_setprio(0);
      // descriptors of this group's next VALU phase (tile t): its DMA issue and its mask
      dma_ks = tiles[toff + min(t + kRing - 1, T - 1)].x;
      mask = t < T ? tiles[toff + t].y : 0;
      }
    } else {
      // VALU phase of tile t: first this group's tile loads (two tiles ahead), then the softmax
      // in base 2, one query per lane. The running max m_run moves only when this tile's max
      // exceeds it by more than 2^kLazy: probabilities stay below 2^kLazy (exact softmax either
      // way, a common shift cancels in O / l) and most tiles skip the rescale.
      tile_dma(dma_ks, (t_valu + kRing - 1) % kRing);
      const bool work = rows_live && p >= 1 + group && t_valu < T;
      if (work) {
        const int lo = mask & 0xffff, hi = mask >> 16;
        if (lo > 0 || hi < kBN) {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int ko = 32 * kb + 8 * (i >> 2) + 4 * g + (i & 3);
              if (ko < lo || ko >= hi) sacc[kb][i] = -INFINITY;
            }
        }
        // tile row max over the lane's 48 scores as a tree of three-input maxima (16 + 5 + 2
        // v_max3), then the other half-wave's value through v_permlane32_swap (no LDS round trip)
        static_assert(NKB == 3, "the max tree is written for 48 scores per lane");
        float m1[16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
          m1[i] = fmaxf(fmaxf(sacc[0][i], sacc[1][i]), sacc[2][i]);
        float m2[6];
#pragma unroll
        for (int i = 0; i < 5; ++i) m2[i] = fmaxf(fmaxf(m1[3 * i], m1[3 * i + 1]), m1[3 * i + 2]);
        m2[5] = m1[15];
        const float mx = fmaxf(fmaxf(fmaxf(m2[0], m2[1]), m2[2]), fmaxf(fmaxf(m2[3], m2[4]), m2[5]));
        const float mt = fmaxf(mx, other_half(mx)) * scale_log2;
        const bool grow = mt > m_run + kLazy;
        if (__any(grow)) {
          const float m_new = grow ? mt : m_run;
          const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
          m_run = m_new;
          l_run *= corr;
#pragma unroll
          for (int m = 0; m < NO; ++m) oacc[m] *= corr;
        }
        // P in bf16 pairs; the row sum adds the bf16 values the PV product uses, two per
        // v_dot2c_f32_bf16 against (1, 1), in four independent chains
        typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
        const bf16x2_t ones = {(__bf16)1.0f, (__bf16)1.0f};
        float rs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; i += 2) {
            const float p0 = __builtin_amdgcn_exp2f(fmaf(sacc[kb][i], scale_log2, -m_run));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(sacc[kb][i + 1], scale_log2, -m_run));
            const uint32_t pk = pack_bf2(p0, p1);
            pb[2 * kb + (i >> 3)][i & 7] = __builtin_bit_cast(__bf16, (uint16_t)(pk & 0xffffu));
            pb[2 * kb + (i >> 3)][(i & 7) + 1] = __builtin_bit_cast(__bf16, (uint16_t)(pk >> 16));
            rs[(i >> 1) & 3] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pk), ones,
                                                               rs[(i >> 1) & 3], false);
          }
        l_run += (rs[0] + rs[1]) + (rs[2] + rs[3]);
      }
    }
    // before an even phase 2(t+1): K(t+1) and V(t) (issued kRing - 1 issues ago by their group)
    // have landed; each group's two latest issues may still be in flight
    if (p & 1) wait_vm_lds<(kRing - 2) * KCG>();
    bare_barrier();
  }

  wait_vm_lds<0>();  // no tile load may land in LDS after the workgroup ends
  store_rows<D>(oacc, l_run, qr, q1, gate, g_row, head, out, o_row, o_head, g);
}

template <int D>
int launch_prepass(const uint16_t *v, int64_t v_row, int64_t v_head, int seq, int heads, void *workspace,
                   hipStream_t stream) {
  const int s_pad = pad_rows(seq);
  hipLaunchKernelGGL(vt_prepass_kernel<D>, dim3(s_pad / 64, heads), dim3(kThreads), 0, stream, v, v_row, v_head,
                     static_cast<uint16_t *>(workspace), seq, s_pad);
  return check_launch("window vt_prepass");
}

// QNORM: q is normalised on load with q_weight / q_eps (see window_attn_kernel)
template <int D, bool QNORM>
int launch_attn(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *k, int64_t k_row, int64_t k_head,
                uint16_t *out, int64_t o_row, int64_t o_head, const uint16_t *gate, int64_t gate_row, int seq,
                int heads, float scale, const int32_t *items, int32_t n_items, const int32_t *tiles,
                const void *workspace, hipStream_t stream, const uint16_t *q_weight = nullptr, float q_eps = 0.f) {
  const int s_pad = pad_rows(seq);
  const int total = n_items * heads;
  const int per_xcd = (total + 7) / 8;
  hipLaunchKernelGGL((window_attn_kernel<D, QNORM>), dim3(per_xcd * 8), dim3(kThreads), 0, stream, q, q_row, q_head, k,
                     k_row, k_head, static_cast<const uint16_t *>(workspace), s_pad, out, o_row, o_head, gate,
                     gate_row, seq, scale * 1.4426950408889634f, reinterpret_cast<const int4 *>(items), n_items,
                     reinterpret_cast<const int2 *>(tiles), per_xcd, total, q_weight, q_eps);
  return check_launch("window_attn");
}

template <int D>
int launch_qkv_prepass(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *q_weight, float q_eps,
                       const uint16_t *k, int64_t k_row, int64_t k_head, const uint16_t *k_weight, float k_eps,
                       const uint16_t *v, int64_t v_row, int64_t v_head, const float *freqs, int64_t f_row, int rot,
                       int seq, int heads, void *workspace, hipStream_t stream) {
  const int s_pad = pad_rows(seq);
  const size_t region = (size_t)heads * D * s_pad;
  uint16_t *vt = static_cast<uint16_t *>(workspace), *kn = vt + region, *qn = vt + 2 * region;
  const dim3 grid((heads + kPrepassHeads - 1) / kPrepassHeads, s_pad / 64);
  if (freqs)
    hipLaunchKernelGGL((qkv_prepass_kernel<D, true>), grid, dim3(kThreads), 0, stream, q, q_row, q_head, q_weight,
                       q_eps, k, k_row, k_head, k_weight, k_eps, v, v_row, v_head, freqs, f_row, rot, vt, kn, qn, seq,
                       s_pad, heads);
  else
    hipLaunchKernelGGL((qkv_prepass_kernel<D, false>), grid, dim3(kThreads), 0, stream, q, q_row, q_head, q_weight,
                       q_eps, k, k_row, k_head, k_weight, k_eps, v, v_row, v_head, freqs, f_row, rot, vt, kn, qn, seq,
                       s_pad, heads);
  return check_launch("window qkv_prepass");
}

int check_rope(const float *freqs, int64_t f_row, int rot, int head_dim) {
  if (!freqs) return VDNH3_OK;
  VDNH3_HOST_CHECK(rot > 0 && rot % 16 == 0 && rot <= head_dim, VDNH3_ERR_INVALID,
                   "rope: rot_dim must be a positive multiple of 16 and at most head_dim %d, got %d", head_dim, rot);
  VDNH3_HOST_CHECK(f_row >= 0 && f_row % 4 == 0 && reinterpret_cast<uintptr_t>(freqs) % 16 == 0, VDNH3_ERR_INVALID,
                   "rope: frequencies must be 16-byte aligned with a row stride multiple of 4");
  return VDNH3_OK;
}

int check_common(int seq, int heads, int head_dim, const void *workspace, size_t workspace_bytes) {
  VDNH3_HOST_CHECK(head_dim == 64 || head_dim == 128, VDNH3_ERR_INVALID,
                   "window attention supports head_dim 64 or 128, got %d", head_dim);
  VDNH3_HOST_CHECK(seq > 0 && heads > 0, VDNH3_ERR_INVALID, "seq and heads must be positive");
  VDNH3_HOST_CHECK(workspace != nullptr && reinterpret_cast<uintptr_t>(workspace) % 16 == 0, VDNH3_ERR_INVALID,
                   "workspace must be non-null and 16-byte aligned");
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
  return size_t(heads) * size_t(head_dim) * size_t(vdnh3::pad_rows(seq)) * sizeof(uint16_t);
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
    return vdnh3::launch_attn<128, false>(q, q_row, q_head, k, k_row, k_head, out, o_row, o_head, gate, gate_row, seq,
                                      heads, scale, items, n_items, tiles, workspace, s);
  return vdnh3::launch_attn<64, false>(q, q_row, q_head, k, k_row, k_head, out, o_row, o_head, gate, gate_row, seq, heads,
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

extern "C" size_t vdnh3_window_norm_workspace_bytes(int seq, int heads, int head_dim, int with_queries) {
  return (with_queries ? 3 : 2) * vdnh3_window_workspace_bytes(seq, heads, head_dim);
}

extern "C" int vdnh3_window_qkv_prepass(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *q_weight,
                                        float q_eps, const uint16_t *k, int64_t k_row, int64_t k_head,
                                        const uint16_t *k_weight, float k_eps, const uint16_t *v, int64_t v_row,
                                        int64_t v_head, const float *freqs, int64_t freqs_row, int rot_dim, int seq,
                                        int heads, int head_dim, void *workspace, size_t workspace_bytes,
                                        void *stream) {
  int rc = vdnh3::check_common(seq, heads, head_dim, workspace, workspace_bytes);
  if (!rc) rc = vdnh3::check_vec(k, k_row, k_head, "k");
  if (!rc) rc = vdnh3::check_vec(v, v_row, v_head, "v");
  if (!rc) rc = vdnh3::check_vec(k_weight, 0, 0, "k_weight");
  if (!rc && q) rc = vdnh3::check_vec(q, q_row, q_head, "q");
  if (!rc && q) rc = vdnh3::check_vec(q_weight, 0, 0, "q_weight");
  if (!rc) rc = vdnh3::check_rope(freqs, freqs_row, rot_dim, head_dim);
  if (rc) return rc;
  const size_t need = vdnh3_window_norm_workspace_bytes(seq, heads, head_dim, q != nullptr);
  VDNH3_HOST_CHECK(workspace_bytes >= need, VDNH3_ERR_INVALID,
                   "workspace of %zu bytes is smaller than the %zu the pre-pass writes", workspace_bytes, need);
  VDNH3_HOST_CHECK(vdnh3::pad_rows(seq) / 64 <= 65535, VDNH3_ERR_INVALID, "the pre-pass supports at most %d rows, got %d",
                   65535 * 64, seq);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return head_dim == 128 ? vdnh3::launch_qkv_prepass<128>(q, q_row, q_head, q_weight, q_eps, k, k_row, k_head,
                                                          k_weight, k_eps, v, v_row, v_head, freqs, freqs_row, rot_dim,
                                                          seq, heads, workspace, s)
                         : vdnh3::launch_qkv_prepass<64>(q, q_row, q_head, q_weight, q_eps, k, k_row, k_head,
                                                         k_weight, k_eps, v, v_row, v_head, freqs, freqs_row, rot_dim,
                                                         seq, heads, workspace, s);
}

extern "C" int vdnh3_window_attn_qnorm(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *q_weight,
                                       float q_eps, uint16_t *out, int64_t o_row, int64_t o_head, const uint16_t *gate,
                                       int64_t gate_row, int seq, int heads, int head_dim, float scale,
                                       const int32_t *items, int32_t n_items, const int32_t *tiles,
                                       const void *workspace, size_t workspace_bytes, void *stream) {
  int rc = vdnh3::check_common(seq, heads, head_dim, workspace, workspace_bytes);
  if (!rc) rc = vdnh3::check_vec(q, q_row, q_head, "q");
  if (!rc) rc = vdnh3::check_vec(q_weight, 0, 0, "q_weight");
  if (rc) return rc;
  VDNH3_HOST_CHECK(workspace_bytes >= vdnh3_window_norm_workspace_bytes(seq, heads, head_dim, 0), VDNH3_ERR_INVALID,
                   "workspace of %zu bytes is smaller than the %zu the normalising attention reads", workspace_bytes,
                   vdnh3_window_norm_workspace_bytes(seq, heads, head_dim, 0));
  VDNH3_HOST_CHECK(out != nullptr && o_row % 4 == 0 && o_head % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 8 == 0,
                   VDNH3_ERR_INVALID, "out must be 8-byte aligned with strides that are multiples of 4 elements");
  VDNH3_HOST_CHECK(items != nullptr && tiles != nullptr && n_items > 0, VDNH3_ERR_INVALID, "empty window plan");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int s_pad = vdnh3::pad_rows(seq);
  // the normalised keys follow the V^T copy in the workspace: [heads][s_pad][head_dim]
  const uint16_t *kn = static_cast<const uint16_t *>(workspace) + (size_t)heads * head_dim * s_pad;
  const int64_t kn_row = head_dim, kn_head = (int64_t)s_pad * head_dim;
  if (head_dim == 128)
    return vdnh3::launch_attn<128, true>(q, q_row, q_head, kn, kn_row, kn_head, out, o_row, o_head, gate, gate_row,
                                         seq, heads, scale, items, n_items, tiles, workspace, s, q_weight, q_eps);
  return vdnh3::launch_attn<64, true>(q, q_row, q_head, kn, kn_row, kn_head, out, o_row, o_head, gate, gate_row, seq,
                                      heads, scale, items, n_items, tiles, workspace, s, q_weight, q_eps);
}
