// K/V short convolutions of the VDN branch features on gfx950 (vdn_h3/runtime.py:319-341,
// vdn_h3/branch.py:443-480, the fused temporal kernel of vdn_h3/kernels.py:100-129):
//   s[f][y][x][c] = bf16( sum_{dy,dx} x[f][y+dy-P][x+dx-P][c] * w_sp[c][dy][dx] )  zero padded, fp32 sum
//   a[f][p][c]    = sum_{dt} s[f+dt-PT][p][c] * w_tm[c][dt]                        zero padded over frames, fp32
//   y = a * sigmoid(a);  with l2norm y /= max(||y||, 1e-6) over the head's D channels;  out = bf16(y)
// The spatial sum is rounded to bf16 because the reference materialises the depthwise Conv2d
// output as a bf16 tensor; the temporal sum, SiLU and norm stay in fp32 up to the one final
// rounding, as in the reference's fused temporal kernel.
//
// One workgroup (1024 threads) owns the D channels of one head on a TX x TY tile of the frame
// grid and walks the frames in order. Per frame it stages the raw tile with its halo in LDS (the
// next frame's loads are in flight during the arithmetic), forms the spatial sums, keeps the last
// KT of them per position in registers (bf16 pairs) and emits the temporal output of frame
// f - KT/2. D/4 lanes share one position, 4 channels (8 bytes) each, so the norm over the head
// is a DPP / swizzle reduction. Taps are bf16 pairs (t, t + 1) and v_dot2_f32_bf16 takes two
// taps of one channel per instruction; one v_perm_b32 re-pairs two staged words by channel. The
// spatial pairs sit in LDS (read once per row and frame), the temporal pairs in registers.
// Workgroups are numbered XCD-aware: the tiles of one head run on one XCD, so the halo rows a
// tile shares with its neighbours come from that XCD's L2 (HBM reads equal the input once).
#include <type_traits>

#include "common.h"

namespace vdnh3 {
namespace {

constexpr int SC_THREADS = 1024;
constexpr int SC_MAX_POS = 64;     // positions of one tile (TX * TY)
constexpr int SC_MAX_STAGE = 160;  // staged positions, tile plus halo ((TX + 2P) * (TY + 2P))

typedef __bf16 sc_bf16x2_t __attribute__((ext_vector_type(2)));
// a.lo * b.lo + a.hi * b.hi + c over bf16 pairs, fp32 accumulate (v_dot2_f32_bf16)
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(sc_bf16x2_t, a), __builtin_bit_cast(sc_bf16x2_t, b), c,
                                         false);
}
// (a.lo, b.lo) and (a.hi, b.hi) of two bf16-pair words, one v_perm_b32 each (selector bytes
// 0-3 pick from the second operand, 4-7 from the first)
__device__ __forceinline__ uint32_t pair_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t pair_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

// sum over aligned groups of L lanes (16 or 32), every lane of a group gets the group's sum:
// DPP quad xor 1, quad xor 2, half-row mirror, row mirror, then a swizzle xor 16
template <int L>
__device__ __forceinline__ float group_sum(float v) {
  auto dpp = [](float x, auto ctrl) __device__ {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xf, 0xf, false));
  };
  v += dpp(v, std::integral_constant<int, 0xb1>{});
  v += dpp(v, std::integral_constant<int, 0x4e>{});
  v += dpp(v, std::integral_constant<int, 0x141>{});
  v += dpp(v, std::integral_constant<int, 0x140>{});
  if constexpr (L == 32) v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f));
  return v;
}

// acc[4] (channels 4 cl .. 4 cl + 3) += sum over the NT taps of staged words src[0 .. NT) (each
// u32x2: channels (0, 1) and (2, 3)) with tap pairs w[pr][channel] (odd last tap zero-padded)
template <int NT>
__device__ __forceinline__ void taps_dot2(const u32x2_t *src, const uint32_t (*w)[4], float *acc) {
#pragma unroll
  for (int pr = 0; pr < (NT + 1) / 2; ++pr) {
#pragma unroll
    for (int wi = 0; wi < 2; ++wi) {
      const uint32_t a = src[2 * pr][wi];
      uint32_t lo = a, hi = a;  // the odd last tap: the raw word against a zero-padded pair
      if (2 * pr + 1 < NT) {
        lo = pair_lo(a, src[2 * pr + 1][wi]);
        hi = pair_hi(a, src[2 * pr + 1][wi]);
      }
      acc[2 * wi] = dot2_bf16(lo, w[pr][2 * wi], acc[2 * wi]);
      acc[2 * wi + 1] = dot2_bf16(hi, w[pr][2 * wi + 1], acc[2 * wi + 1]);
    }
  }
}

// tap pairs of channel j (0..3 within a lane's 4) from NT bf16 taps: (t, t + 1) per pair, the
// odd last tap on the half of its channel's position in the staged word
template <int NT>
__device__ __forceinline__ void load_tap_pairs(const uint16_t *taps, int j, uint32_t (*w)[4]) {
#pragma unroll
  for (int pr = 0; pr < NT / 2; ++pr)
    w[pr][j] = (uint32_t)taps[2 * pr] | ((uint32_t)taps[2 * pr + 1] << 16);
  if constexpr (NT & 1) {
    const uint32_t last = taps[NT - 1];
    w[NT / 2][j] = (j & 1) ? last << 16 : last;
  }
}

// up to four tensors of one frame grid convolved by one launch (e.g. k and v): their workgroups
// fill the same rounds instead of each launch ending on a partly empty one
constexpr int SC_MAX_JOBS = 4;
struct ConvJob {
  const uint16_t *x;
  int64_t x_row, x_head;
  const uint16_t *w_sp, *w_tm;
  int l2norm;
  uint16_t *out;
  int64_t o_row, o_head;
};
struct ConvJobs {
  ConvJob j[SC_MAX_JOBS];
};

template <int D, int KS, int KT>
__global__ __launch_bounds__(SC_THREADS) void short_conv_kernel(ConvJobs jobs, int F, int gh, int gw, int TX, int TY,
                                                                 int nx, int n_tiles, int heads) {
  constexpr int P = KS / 2, PT = KT / 2;
  constexpr int LPP = D / 4;                      // lanes per position
  constexpr int PPP = SC_THREADS / LPP;           // positions per pass
  constexpr int NPASS = SC_MAX_POS / PPP;         // passes over a tile
  constexpr int CPP = D / 8;                      // 16-byte chunks per staged position
  constexpr int MAXL = (SC_MAX_STAGE * CPP + SC_THREADS - 1) / SC_THREADS;
  __shared__ __attribute__((aligned(16))) uint16_t tile[SC_MAX_STAGE * D];

  // XCD-aware numbering: dispatch deals workgroups to the 8 XCDs round-robin; XCD x takes the
  // x-th contiguous run of the logical order (head-major), so a head's tiles share one L2
  const int nb = gridDim.x, per = nb >> 3, rem = nb & 7, xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int logical = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
  const int job = logical / (heads * n_tiles), hti = logical - job * heads * n_tiles;
  const int h = hti / n_tiles, ti = hti - h * n_tiles;
  const ConvJob &J = jobs.j[job];
  const uint16_t *__restrict__ x = J.x;
  const uint16_t *__restrict__ w_sp = J.w_sp;
  const uint16_t *__restrict__ w_tm = J.w_tm;
  uint16_t *__restrict__ out = J.out;
  const int64_t x_row = J.x_row, x_head = J.x_head, o_row = J.o_row, o_head = J.o_head;
  const int l2norm = J.l2norm;
  const int y0 = (ti / nx) * TY, x0 = (ti % nx) * TX;
  const int tid = threadIdx.x, cl = tid % LPP, ps = tid / LPP;
  const int SX = TX + 2 * P, SY = TY + 2 * P, n_stage = SX * SY * CPP;
  const int T = gh * gw;

  // filter taps of this lane's 4 channels: spatial as bf16 pairs (dx, dx + 1) per row, the odd
  // last tap of a row paired with zero on the side of the other channel of its staged word
  // (dot2 of the raw word then picks this channel); temporal in fp32
  // The spatial pairs live in LDS as [dy][pair][lane group cl][4 channels] (one 16-byte read per
  // pair and row, consecutive across cl), the temporal pairs in registers.
  constexpr int NPR = (KS + 1) / 2;
  __shared__ __attribute__((aligned(16))) uint32_t wlds[KS * NPR * LPP * 4];
  if (tid < LPP) {
    uint32_t row[NPR][4];
#pragma unroll
    for (int dy = 0; dy < KS; ++dy) {
#pragma unroll
      for (int j = 0; j < 4; ++j) load_tap_pairs<KS>(w_sp + (((int64_t)h * D + 4 * tid + j) * KS + dy) * KS, j, row);
#pragma unroll
      for (int pr = 0; pr < NPR; ++pr)
        *reinterpret_cast<u32x4_t *>(wlds + ((dy * NPR + pr) * LPP + tid) * 4) =
            u32x4_t{row[pr][0], row[pr][1], row[pr][2], row[pr][3]};
    }
  }
  uint32_t wtm[(KT + 1) / 2][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) load_tap_pairs<KT>(w_tm + ((int64_t)h * D + 4 * cl + j) * KT, j, wtm);

  // this thread's tile positions (one per pass); slots past the tile read position 0
  int lbase[NPASS];
  int64_t obase[NPASS];
  bool valid[NPASS];
#pragma unroll
  for (int i = 0; i < NPASS; ++i) {
    const int pi = i * PPP + ps;
    const bool in_tile = pi < TX * TY;
    const int py = in_tile ? pi / TX : 0, px = in_tile ? pi % TX : 0;
    valid[i] = in_tile && y0 + py < gh && x0 + px < gw;
    lbase[i] = (py * SX + px) * D + 4 * cl;
    obase[i] = valid[i] ? (int64_t)((y0 + py) * gw + x0 + px) * o_row + (int64_t)h * o_head + 4 * cl : 0;
  }

  // staging of frame f: chunk e = position (ly, lx) of the tile plus halo, 16-byte piece e % CPP;
  // its element offset inside a frame is the same for every frame (-1: outside the grid, zero)
  int soff[MAXL];
#pragma unroll
  for (int u = 0; u < MAXL; ++u) {
    const int e = tid + u * SC_THREADS;
    soff[u] = -1;
    if (e < n_stage) {
      const int sp = e / CPP, ch = e - sp * CPP, ly = sp / SX, lx = sp - ly * SX;
      const int gy = y0 + ly - P, gx = x0 + lx - P;
      if (gy >= 0 && gy < gh && gx >= 0 && gx < gw) soff[u] = (gy * gw + gx) * (int)x_row + 8 * ch;
    }
  }
  u32x4_t pre[MAXL];
  auto stage_load = [&](int f) __device__ {
    const uint16_t *xf = x + (int64_t)f * T * x_row + (int64_t)h * x_head;
#pragma unroll
    for (int u = 0; u < MAXL; ++u) pre[u] = soff[u] >= 0 ? ld16(xf + soff[u]) : u32x4_t{0, 0, 0, 0};
  };
  auto stage_store = [&]() __device__ {
#pragma unroll
    for (int u = 0; u < MAXL; ++u) {
      const int e = tid + u * SC_THREADS;
      if (e < n_stage) st16(tile + 8 * e, pre[u]);
    }
  };

  uint32_t ring[NPASS][KT][2];
#pragma unroll
  for (int i = 0; i < NPASS; ++i)
#pragma unroll
    for (int t = 0; t < KT; ++t) ring[i][t][0] = ring[i][t][1] = 0u;

  stage_load(0);
  for (int f = 0; f < F + PT; ++f) {
    uint32_t fresh[NPASS][2];
    if (f < F) {
      __syncthreads();  // every lane is done reading the previous frame's tile
      stage_store();
      __syncthreads();
      if (f + 1 < F) stage_load(f + 1);
      float acc[NPASS][4];
#pragma unroll
      for (int i = 0; i < NPASS; ++i) acc[i][0] = acc[i][1] = acc[i][2] = acc[i][3] = 0.f;
#pragma unroll
      for (int dy = 0; dy < KS; ++dy) {
        uint32_t wr[NPR][4];
#pragma unroll
        for (int pr = 0; pr < NPR; ++pr) {
          const u32x4_t w4 = *reinterpret_cast<const u32x4_t *>(wlds + ((dy * NPR + pr) * LPP + cl) * 4);
          wr[pr][0] = w4[0], wr[pr][1] = w4[1], wr[pr][2] = w4[2], wr[pr][3] = w4[3];
        }
#pragma unroll
        for (int i = 0; i < NPASS; ++i) {
          u32x2_t v[KS];
#pragma unroll
          for (int dx = 0; dx < KS; ++dx)
            v[dx] = *reinterpret_cast<const u32x2_t *>(tile + lbase[i] + (dy * SX + dx) * D);
          taps_dot2<KS>(v, wr, acc[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < NPASS; ++i) {
        fresh[i][0] = pack_bf2(acc[i][0], acc[i][1]);
        fresh[i][1] = pack_bf2(acc[i][2], acc[i][3]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NPASS; ++i) fresh[i][0] = fresh[i][1] = 0u;
    }
    // ring[i][t] holds the spatial sum of frame f - KT + 1 + t
#pragma unroll
    for (int i = 0; i < NPASS; ++i) {
#pragma unroll
      for (int t = 0; t + 1 < KT; ++t) {
        ring[i][t][0] = ring[i][t + 1][0];
        ring[i][t][1] = ring[i][t + 1][1];
      }
      ring[i][KT - 1][0] = fresh[i][0];
      ring[i][KT - 1][1] = fresh[i][1];
    }
    const int fo = f - PT;  // output frame: its taps are frames fo - PT .. fo + PT = ring[0 .. KT-1]
    if (fo < 0) continue;
#pragma unroll
    for (int i = 0; i < NPASS; ++i) {
      float a[4] = {0.f, 0.f, 0.f, 0.f};
      u32x2_t r[KT];
#pragma unroll
      for (int t = 0; t < KT; ++t) r[t] = u32x2_t{ring[i][t][0], ring[i][t][1]};
      taps_dot2<KT>(r, wtm, a);
      // SiLU and the norm with the hardware exp2 / reciprocal (a few fp32 ulps, far below the
      // one bf16 rounding of the output)
      float y[4], ss = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        y[j] = a[j] * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(a[j] * -1.44269504088896341f));
        ss = fmaf(y[j], y[j], ss);
      }
      if (l2norm) {
        // 1 / max(||y||, 1e-6) = rsqrt(max(||y||^2, 1e-12))
        const float inv = __builtin_amdgcn_rsqf(fmaxf(group_sum<LPP>(ss), 1e-12f));
#pragma unroll
        for (int j = 0; j < 4; ++j) y[j] *= inv;
      }
      if (valid[i])
        *reinterpret_cast<u32x2_t *>(out + obase[i] + (int64_t)fo * T * o_row) =
            u32x2_t{pack_bf2(y[0], y[1]), pack_bf2(y[2], y[3])};
    }
  }
}

// Tile shape of the frame grid: the fewest tiles with TX * TY <= 64 positions, TX, TY <= 16
// and the tile plus its halo within the LDS stage.
void pick_tile(int gh, int gw, int P, int *TX, int *TY, int *nx, int *ny) {
  int best = -1;
  for (int tx = 1; tx <= 16; ++tx) {
    const int cx = (gw + tx - 1) / tx, txr = (gw + cx - 1) / cx;
    int ty = SC_MAX_POS / txr;
    if (ty > 16) ty = 16;
    while (ty > 1 && (txr + 2 * P) * (ty + 2 * P) > SC_MAX_STAGE) --ty;
    if ((txr + 2 * P) * (ty + 2 * P) > SC_MAX_STAGE) continue;
    const int cy = (gh + ty - 1) / ty, tyr = (gh + cy - 1) / cy;
    const int cost = cx * cy;
    if (best < 0 || cost < best) {
      best = cost;
      *TX = txr;
      *TY = tyr;
      *nx = cx;
      *ny = cy;
    }
  }
}

template <int D, int KS, int KT>
void launch(const ConvJobs &jobs, int n_jobs, int F, int gh, int gw, int heads, hipStream_t s) {
  int TX = 1, TY = 1, nx = gw, ny = gh;
  pick_tile(gh, gw, KS / 2, &TX, &TY, &nx, &ny);
  const int n_tiles = nx * ny;
  hipLaunchKernelGGL((short_conv_kernel<D, KS, KT>), dim3(n_jobs * heads * n_tiles), dim3(SC_THREADS), 0, s, jobs, F,
                     gh, gw, TX, TY, nx, n_tiles, heads);
}

int run_jobs(const vdnh3_short_conv_job *jobs, int n_jobs, int kernel_h, int kernel_w, int kernel_t, int frames,
             int grid_h, int grid_w, int heads, int head_dim, hipStream_t s) {
  VDNH3_HOST_CHECK(jobs && n_jobs >= 1 && n_jobs <= SC_MAX_JOBS, VDNH3_ERR_INVALID,
                   "short_conv: 1 to %d tensors per launch, got %d", SC_MAX_JOBS, n_jobs);
  VDNH3_HOST_CHECK(head_dim == 64 || head_dim == 128, VDNH3_ERR_INVALID,
                   "short_conv: head_dim must be 64 or 128, got %d", head_dim);
  VDNH3_HOST_CHECK(kernel_h == kernel_w && (kernel_h == 3 || kernel_h == 5) && (kernel_t == 3 || kernel_t == 5),
                   VDNH3_ERR_INVALID,
                   "short_conv: supported kernels are 3x3 or 5x5 spatial and 3 or 5 temporal taps, got %dx%d and %d",
                   kernel_h, kernel_w, kernel_t);
  VDNH3_HOST_CHECK(frames > 0 && grid_h > 0 && grid_w > 0 && heads > 0, VDNH3_ERR_INVALID,
                   "short_conv: empty frame grid or no heads");
  ConvJobs cj{};
  for (int i = 0; i < n_jobs; ++i) {
    const vdnh3_short_conv_job &j = jobs[i];
    VDNH3_HOST_CHECK(j.x && j.w_spatial && j.w_temporal && j.out, VDNH3_ERR_INVALID, "short_conv: null operand");
    VDNH3_HOST_CHECK(j.x_row % 8 == 0 && j.x_head % 8 == 0 && reinterpret_cast<uintptr_t>(j.x) % 16 == 0,
                     VDNH3_ERR_INVALID, "short_conv: x must be 16-byte aligned with strides multiple of 8");
    VDNH3_HOST_CHECK((int64_t)grid_h * grid_w * j.x_row < ((int64_t)1 << 31), VDNH3_ERR_INVALID,
                     "short_conv: one frame of x must span fewer than 2^31 elements");
    VDNH3_HOST_CHECK(j.out_row % 4 == 0 && j.out_head % 4 == 0 && reinterpret_cast<uintptr_t>(j.out) % 8 == 0,
                     VDNH3_ERR_INVALID, "short_conv: out must be 8-byte aligned with strides multiple of 4");
    cj.j[i] = ConvJob{j.x, j.x_row, j.x_head, j.w_spatial, j.w_temporal, j.l2norm, j.out, j.out_row, j.out_head};
  }
#define VDNH3_SC(D, KS, KT) \
  if (head_dim == D && kernel_h == KS && kernel_t == KT) launch<D, KS, KT>(cj, n_jobs, frames, grid_h, grid_w, heads, s);
  VDNH3_SC(128, 5, 5)
  VDNH3_SC(128, 5, 3)
  VDNH3_SC(128, 3, 5)
  VDNH3_SC(128, 3, 3)
  VDNH3_SC(64, 5, 5)
  VDNH3_SC(64, 5, 3)
  VDNH3_SC(64, 3, 5)
  VDNH3_SC(64, 3, 3)
#undef VDNH3_SC
  return check_launch("short_conv");
}

}  // namespace
}  // namespace vdnh3

extern "C" int vdnh3_short_conv(const uint16_t *x, int64_t x_row, int64_t x_head, const uint16_t *w_spatial,
                                int kernel_h, int kernel_w, const uint16_t *w_temporal, int kernel_t, int frames,
                                int grid_h, int grid_w, int heads, int head_dim, int l2norm, uint16_t *out,
                                int64_t out_row, int64_t out_head, void *stream) {
  const vdnh3_short_conv_job job{x, x_row, x_head, w_spatial, w_temporal, l2norm, out, out_row, out_head};
  return vdnh3::run_jobs(&job, 1, kernel_h, kernel_w, kernel_t, frames, grid_h, grid_w, heads, head_dim,
                         static_cast<hipStream_t>(stream));
}

extern "C" int vdnh3_short_conv_batch(const vdnh3_short_conv_job *jobs, int n_jobs, int kernel_h, int kernel_w,
                                      int kernel_t, int frames, int grid_h, int grid_w, int heads, int head_dim,
                                      void *stream) {
  return vdnh3::run_jobs(jobs, n_jobs, kernel_h, kernel_w, kernel_t, frames, grid_h, grid_w, heads, head_dim,
                         static_cast<hipStream_t>(stream));
}
