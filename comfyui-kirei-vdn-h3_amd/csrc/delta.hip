// Video Delta Attention (the VDN linear branch) on gfx950.
//
// Per frame f and head h, with k~ = L2(SiLU(k)), v~ = SiLU(v), q~ = L2(SiLU(q)) (vdn_h3/kernels.py:47-51):
//   frame_stats : A = k~^T diag(beta) k~ (fp32, symmetrised), B = bf16((v~ * beta)^T k~)      (vdn_h3/branch.py:197-243)
//   factor      : L = chol(I + A), W = L^-1, M = W^T W, Phi = diag(alpha) M, J = B M, info       (vdn_h3/branch.py:62-71, :148-160)
//   scan        : P_f = J_f + P_{f-1} Phi_f forward, Q_f = J_f + Q_{f+1} Phi_f backward         (vdn_h3/runtime.py:118-131)
//   readout     : L_f = decayed P[lo-1] + Q[hi+1] (bf16), r = q~ L_f^T (bf16), y = RMSNorm(r) w * gate
//                 (vdn_h3/branch.py:372-396, vdn_h3/runtime.py:406-419, vdn_h3/branch.py:494-505)
// plus the small per-frame pieces: frame means, the fp32 alpha projections and decay (vdn_h3/branch.py:483-491).
//
// The dtype contract follows the reference's bf16 model: features, beta, B, the gathered state,
// the readout and every epilogue step are rounded to bf16 where the reference materialises a
// bf16 tensor; A, the factor, the scans and the gather run in fp32.
#include <algorithm>

#include "common.h"

namespace vdnh3 {
namespace {

// bf16(s / n) as fp32, bit-identical to round_bf(s / n); rn = 1 / n (correctly rounded), so
// s * rn is within 1.5 ulp of the quotient.
__device__ __forceinline__ float div_bf(float s, float n, float rn) {
  const float y = s * rn;
  if (__builtin_expect(near_bf16_midpoint(y), 0)) return round_bf(s / n);
  return round_bf(y);
}

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ f32x16_t mfma_f32_32x32x2(float a, float b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------------------
// frame statistics. grid = frames * heads, 256 threads. Tokens are consumed in tiles of 32,
// stored transposed ([d][t]) in LDS so both MFMA operands read 8 consecutive tokens; the LDS
// tiles are double-buffered (one barrier per tile) and each tile's raw k / v / beta are loaded
// into registers while the previous tile's features are formed and multiplied.
// A's operand beta*k~ (exact in fp32: a product of two bf16 values) is split into
// hi = bf16(x) and lo = x - hi, both exact bf16, so A = hi^T k~ + lo^T k~ carries every bit.
// KF / VF: k / v already hold the features k~ / v~ (the output of the short convolutions),
// so the feature map is not applied on load.
// AB: A in bf16 as the reference computes it with a_fp32=False (vdn_h3/branch.py:238-240):
// S = bf16(hi^T k~) (the bf16 product of bf16(k~ * beta) and k~, fp32 accumulation), then
// 0.5 (S + S^T) in fp32; the lo half and its MFMAs are skipped.
template <int D, bool KF, bool VF, bool AB>
__global__ __launch_bounds__(256, 2) void frame_stats_kernel(const uint16_t *__restrict__ k, int64_t k_row,
                                                             int64_t k_head, const uint16_t *__restrict__ v,
                                                             int64_t v_row, int64_t v_head,
                                                             const uint16_t *__restrict__ beta, int64_t beta_row,
                                                             int T, int heads, float *__restrict__ A_out,
                                                             float *__restrict__ B_out) {
  constexpr int TT = 32, P = TT + 8, CH = D / 8, NB = D / 64;
  constexpr int TILE = D * P;
  constexpr int BUF_BYTES = 4 * TILE * 2, SYM_BYTES = D * (D + 1) * 4;
  constexpr int LDS_BYTES = 2 * BUF_BYTES > SYM_BYTES ? 2 * BUF_BYTES : SYM_BYTES;
  __shared__ __attribute__((aligned(16))) uint8_t smem[LDS_BYTES];

  const int fh = blockIdx.x, f = fh / heads, h = fh - f * heads;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int wm = (wave >> 1) * 32 * NB, wn = (wave & 1) * 32 * NB;
  const int p = tid / CH, c = tid % CH;  // loader: token pair p, 16-byte chunk c of the row
  const bool loader = p < TT / 2;
  const int64_t row0 = (int64_t)f * T;

  f32x16_t accA[NB][NB], accB[NB][NB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) accA[i][j] = accB[i][j] = f32x16_t{};

  // raw operands of one tile for this loader thread: tokens t0 + 2p, t0 + 2p + 1
  struct Raw {
    u32x4_t k[2], v[2];
    float b[2];
  };
  auto load_raw = [&](Raw &r, int t0) __device__ {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int t = t0 + 2 * p + e;
      r.k[e] = r.v[e] = u32x4_t{0, 0, 0, 0};
      r.b[e] = 0.f;
      if (loader && t < T) {
        r.k[e] = ld16(k + (row0 + t) * k_row + (int64_t)h * k_head + 8 * c);
        r.v[e] = ld16(v + (row0 + t) * v_row + (int64_t)h * v_head + 8 * c);
        r.b[e] = bf2f(beta[(row0 + t) * beta_row + h]);
      }
    }
  };
  // LDS tile layout [d][token]: 8-token group tg of row d sits at group slot tg ^ ((d / 8) % 4),
  // which spreads the transposed writes of one instruction over 4x more banks
  auto tile_step = [&](Raw &r, int t0, int buf) __device__ {
    uint16_t *Kt = reinterpret_cast<uint16_t *>(smem + buf * BUF_BYTES);
    uint16_t *Xh = Kt + TILE;
    uint16_t *Xl = Xh + TILE;
    uint16_t *Vb = Xl + TILE;
    if (loader) {
      // features of this tile from the registers, then the next tile's loads
      uint32_t kk[2][8], xh[2][8], xl[2][8], vb[2][8];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        float sv[8], sumsq = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t w = r.k[e][j >> 1];
          const float raw = (j & 1) ? bf_hi(w) : bf_lo(w);
          sv[j] = KF ? raw : silu_bf(raw);
          sumsq += sv[j] * sv[j];
        }
        float nrm = 1.f, rn = 1.f;
        if (!KF) {
#pragma unroll
          for (int o = 1; o < CH; o <<= 1) sumsq += __shfl_xor(sumsq, o);
          nrm = fmaxf(round_bf(sqrtf(sumsq)), 1e-6f);
          rn = 1.f / nrm;
        }
        const float b = r.b[e];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float kt = KF ? sv[j] : div_bf(sv[j], nrm, rn);
          const float x = kt * b;  // exact
          const float hi = round_bf(x);
          kk[e][j] = f2bf(kt);
          xh[e][j] = f2bf(hi);
          if (!AB) xl[e][j] = f2bf(x - hi);
          const uint32_t w = r.v[e][j >> 1];
          const float vr = (j & 1) ? bf_hi(w) : bf_lo(w);
          vb[e][j] = f2bf((VF ? vr : silu_bf(vr)) * b);
        }
      }
      if (t0 + TT < T) load_raw(r, t0 + TT);
      const int col = 8 * ((p >> 2) ^ (c & 3)) + 2 * (p & 3);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int o = (8 * c + j) * P + col;
        *reinterpret_cast<uint32_t *>(Kt + o) = kk[0][j] | (kk[1][j] << 16);
        *reinterpret_cast<uint32_t *>(Xh + o) = xh[0][j] | (xh[1][j] << 16);
        if (!AB) *reinterpret_cast<uint32_t *>(Xl + o) = xl[0][j] | (xl[1][j] << 16);
        *reinterpret_cast<uint32_t *>(Vb + o) = vb[0][j] | (vb[1][j] << 16);
      }
    }
    // one barrier: this tile is complete, and every wave is done with the buffer the next
    // tile will overwrite (it was read two tiles ago, before the previous barrier)
    __syncthreads();
    const int sw = (l32 >> 3) & 3;  // rows 32 i + l32 share (row / 8) % 4
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int slot = 8 * ((2 * ks + g) ^ sw);
      bf16x8_t ah[NB], al[NB], av[NB], bk[NB];
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int ro = (wm + 32 * i + l32) * P + slot;
        ah[i] = as_bf16x8(ld16(Xh + ro));
        if (!AB) al[i] = as_bf16x8(ld16(Xl + ro));
        av[i] = as_bf16x8(ld16(Vb + ro));
        bk[i] = as_bf16x8(ld16(Kt + (wn + 32 * i + l32) * P + slot));
      }
#pragma unroll
      for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          accA[i][j] = mfma_bf16_32x32x16(ah[i], bk[j], accA[i][j]);
          if (!AB) accA[i][j] = mfma_bf16_32x32x16(al[i], bk[j], accA[i][j]);
          accB[i][j] = mfma_bf16_32x32x16(av[i], bk[j], accB[i][j]);
        }
    }
  };

  Raw r;
  load_raw(r, 0);
  int buf = 0;
  for (int t0 = 0; t0 < T; t0 += TT, buf ^= 1) tile_step(r, t0, buf);
  __syncthreads();  // the symmetrisation below reuses the tile buffers

  // A -> LDS, then 0.5 (A + A^T); B rounded to bf16 like the reference's bf16 matmul output
  float *S = reinterpret_cast<float *>(smem);
  float *Bo = B_out + (int64_t)fh * D * D;
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = wm + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3), n = wn + 32 * j + l32;
        S[m * (D + 1) + n] = AB ? round_bf(accA[i][j][r]) : accA[i][j][r];
        Bo[m * D + n] = round_bf(accB[i][j][r]);
      }
  __syncthreads();
  float *Ao = A_out + (int64_t)fh * D * D;
  for (int e = tid; e < D * D; e += 256) {
    const int m = e / D, n = e - m * D;
    Ao[e] = 0.5f * (S[m * (D + 1) + n] + S[n * (D + 1) + m]);
  }
}

// ---------------------------------------------------------------------------------------
// factor. grid = n matrices, 256 threads. M = (I + A)^-1 by the symmetric sweep operator: the
// working matrix S starts as I + A and is swept on pivots k = 0 .. D-1,
//   d = S[k][k];  S[i][l] -= S[i][k] S[k][l] / d;  S[i][k] = S[k][i] = S[i][k] / d;  S[k][k] = -1 / d
// (i, l != k), which leaves S = -(I + A)^-1 and keeps S symmetric throughout. Pivot k is the
// k-th leading Schur complement - the square of Cholesky's L[k][k] - so the first pivot that
// is not positive marks the leading minor of order k + 1 that is not positive-definite, the
// condition the reference's Cholesky reports. Each thread keeps a (D/16) x (D/16) sub-block of
// S in registers (a 16 x 16 grid of sub-blocks); column k of each step is broadcast through a
// double-buffered LDS line (one barrier per pivot). Then Phi = diag(alpha) M from registers and
// J = B M on v_mfma_f32_32x32x2_f32.
template <int D>
__global__ __launch_bounds__(256) void factor_kernel(const float *__restrict__ A, const float *__restrict__ B,
                                                     const float *__restrict__ alpha, float *__restrict__ Phi,
                                                     float *__restrict__ J, float j_scale, int *__restrict__ info) {
  constexpr int SB = D / 16, PITCH = D + 1, NBW = D / 64;  // NBW: 32x32 blocks per wave side
  __shared__ float Lb[D * PITCH];
  __shared__ __attribute__((aligned(16))) float bcast[2][D];
  const int mat = blockIdx.x, tid = threadIdx.x;
  const int ib = tid >> 4, kb0 = tid & 15;  // sub-block row / column of this thread
  const int i0 = ib * SB, k0 = kb0 * SB;
  const float *Am = A + (int64_t)mat * D * D;

  float S[SB][SB];
#pragma unroll
  for (int a = 0; a < SB; ++a)
#pragma unroll
    for (int b = 0; b < SB; ++b) S[a][b] = Am[(i0 + a) * D + k0 + b] + ((i0 + a) == (k0 + b) ? 1.f : 0.f);

  int fail = 0;
  for (int kb = 0; kb < 16 && !fail; ++kb) {
#pragma unroll
    for (int b = 0; b < SB; ++b) {
      const int k = kb * SB + b;
      float *col = bcast[k & 1];
      if (kb0 == kb) {
#pragma unroll
        for (int a = 0; a < SB; ++a) col[i0 + a] = S[a][b];
      }
      __syncthreads();
      const float d = col[k];
      if (!(d > 0.f)) {  // uniform: every thread reads the same pivot
        fail = k + 1;
        break;
      }
      const float rd = 1.f / d;
      float ci[SB], ck[SB];
#pragma unroll
      for (int a = 0; a < SB; ++a) ci[a] = col[i0 + a] * rd;
#pragma unroll
      for (int c = 0; c < SB; ++c) ck[c] = col[k0 + c];
#pragma unroll
      for (int a = 0; a < SB; ++a)
#pragma unroll
        for (int c = 0; c < SB; ++c) S[a][c] = fmaf(-ci[a], ck[c], S[a][c]);
      // row and column k: S[i][k] = S[k][i] = S[i][k] / d, S[k][k] = -1 / d
      if (kb0 == kb) {
#pragma unroll
        for (int a = 0; a < SB; ++a) S[a][b] = ci[a];
      }
      if (ib == kb) {
#pragma unroll
        for (int c = 0; c < SB; ++c) S[b][c] = ck[c] * rd;
        if (kb0 == kb) S[b][b] = -rd;
      }
    }
  }
  if (tid == 0) info[mat] = fail;

  // M = -S: Phi = diag(alpha) M straight from registers, M into LDS for J = B M
  float *Pm = Phi ? Phi + (int64_t)mat * D * D : nullptr;
  const float *al = alpha ? alpha + (int64_t)mat * D : nullptr;
#pragma unroll
  for (int a = 0; a < SB; ++a) {
    const float sa = al ? -al[i0 + a] : -1.f;
#pragma unroll
    for (int c = 0; c < SB; ++c) {
      Lb[(i0 + a) * PITCH + k0 + c] = -S[a][c];
      if (Pm) Pm[(i0 + a) * D + k0 + c] = sa * S[a][c];
    }
  }
  __syncthreads();
  const int wave = tid >> 6, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int wm = (wave >> 1) * 32 * NBW, wn = (wave & 1) * 32 * NBW;
  f32x16_t acc[NBW][NBW];

  // J = B Minv: lane group g contracts over k in [g*D/2, (g+1)*D/2); B rows stream from memory
  const float *Bm = B + (int64_t)mat * D * D;
#pragma unroll
  for (int i = 0; i < NBW; ++i)
#pragma unroll
    for (int j = 0; j < NBW; ++j) acc[i][j] = f32x16_t{};
  for (int s0 = 0; s0 < D / 2; s0 += 4) {
    f32x4_t brow[NBW];
#pragma unroll
    for (int i = 0; i < NBW; ++i)
      brow[i] = *reinterpret_cast<const f32x4_t *>(Bm + (wm + 32 * i + l32) * D + g * (D / 2) + s0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int kappa = g * (D / 2) + s0 + e;
      float bv[NBW];
#pragma unroll
      for (int j = 0; j < NBW; ++j) bv[j] = Lb[kappa * PITCH + wn + 32 * j + l32];
#pragma unroll
      for (int i = 0; i < NBW; ++i)
#pragma unroll
        for (int j = 0; j < NBW; ++j) acc[i][j] = mfma_f32_32x32x2(brow[i][e], bv[j], acc[i][j]);
    }
  }
  float *Jm = J + (int64_t)mat * D * D;
#pragma unroll
  for (int i = 0; i < NBW; ++i)
#pragma unroll
    for (int j = 0; j < NBW; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = wm + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3), n = wn + 32 * j + l32;
        Jm[m * D + n] = j_scale * acc[i][j][r];
      }
}

// ---------------------------------------------------------------------------------------
// scan. grid = heads * 2 directions * D/32 row blocks; D/32 wavefronts, wavefront w owns state
// columns [32w, 32w+32). The state is kept transposed, X = P^T, so the 32x32 accumulator of
// one step (lane = state row) is the next step's B operand after one LDS exchange:
//   X_f = Phi_f^T X_{f-1} + J_f^T
template <int D>
__global__ __launch_bounds__(64 * (D / 32)) void scan_kernel(const float *__restrict__ Phi, const float *__restrict__ J,
                                                             const float *__restrict__ init,
                                                             float *__restrict__ prefix, float *__restrict__ suffix,
                                                             int F, int heads) {
  constexpr int NRB = D / 32, PITCH = 32 + 4;
  __shared__ float St[2][D * PITCH];
  const int bid = blockIdx.x;
  const int rb = bid % NRB, dir = (bid / NRB) & 1, h = bid / (2 * NRB);
  const int tid = threadIdx.x, cb = tid >> 6, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int r0 = rb * 32;
  for (int e = tid; e < D * 32; e += 64 * NRB) {
    const int c = e >> 5, r = e & 31;
    St[0][c * PITCH + r] = init ? init[((int64_t)h * D + r0 + r) * D + c] : 0.f;
  }
  __syncthreads();
  float *out = dir == 0 ? prefix : suffix;
  int cur = 0;
  for (int step = 0; step < F; ++step) {
    const int f = dir == 0 ? step : F - 1 - step;
    const int64_t base = ((int64_t)f * heads + h) * D * D;
    const float *Pf = Phi + base;
    f32x16_t acc = f32x16_t{};
#pragma unroll 16
    for (int s = 0; s < D / 2; ++s) {
      const int kappa = 2 * s + g;
      acc = mfma_f32_32x32x2(Pf[kappa * D + 32 * cb + l32], St[cur][kappa * PITCH + l32], acc);
    }
    const float *Jr = J + base + (int64_t)(r0 + l32) * D;
    float *Or = out + base + (int64_t)(r0 + l32) * D;
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const int c0 = 32 * cb + 8 * i4 + 4 * g;
      const f32x4_t jv = *reinterpret_cast<const f32x4_t *>(Jr + c0);
      f32x4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] = acc[4 * i4 + e] + jv[e];
        St[cur ^ 1][(c0 + e) * PITCH + l32] = o[e];
      }
      *reinterpret_cast<f32x4_t *>(Or + c0) = o;
    }
    __syncthreads();
    cur ^= 1;
  }
}

// ---------------------------------------------------------------------------------------
// Running sums of log(alpha) over frames: out[i][h][d] = sum_{j < i} log(max(alpha[j][h][d],
// 1e-12)), i = 0 .. F, summed in frame order (the decay factors of the readout are
// differences of these). One thread per (h, d).
__global__ void alpha_logsum_kernel(const float *__restrict__ alpha, float *__restrict__ out, int F, int hd) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= hd) return;
  float lp = 0.f;
  out[e] = 0.f;
  for (int i = 0; i < F; ++i) {
    lp += logf(fmaxf(alpha[(int64_t)i * hd + e], 1e-12f));
    out[(int64_t)(i + 1) * hd + e] = lp;
  }
}

// ---------------------------------------------------------------------------------------
// readout. grid = frame_count * heads, 256 threads; wavefronts take 32-token tiles in turn. The grid
// covers frames f0 .. f0 + frame_count - 1 of the F frames the banks and bounds describe; the rows of
// q, the gate and out are those of that range (frame f's tokens at rows (f - f0) T ..).
//   L_f[v][k] = bf16(before[v][k] * decay_b[k] + after[v][k] * decay_a[k])   (LDS, [v][k])
//   r^T = L_f q~^T on bf16 MFMA (lane = token, so the RMS over v is in-lane plus one exchange)
// The normalised, weighted tile y (bf16) goes through a per-wavefront LDS stage so that the
// gate is read and the output written as row-contiguous 16-byte pieces; the tile's gate rows
// are loaded before its MFMAs, the next tile's q after its features.
// QF: q already holds the features q~ (the output of a short convolution).
// FG: the output gate is computed here, gate = bf16(sigmoid(bf16(gate_hidden W_up^T + b_up))) for
// this head's D columns (vdn_h3/branch.py:754-758), as MFMAs beside r: W_up's head slice and the
// bias sit in LDS in place of the y stage, and the output leaves from the accumulator layout.
struct ReadoutGate {
  const uint16_t *gate;    // !FG: [rows][heads * D] bf16
  int64_t gate_row;
  const uint16_t *hidden;  // FG: [rows][D] bf16 (x W_down^T)
  int64_t hidden_row;
  const uint16_t *w_up;    // FG: [heads * D][D] bf16
  const uint16_t *b_up;    // FG: [heads * D] bf16 or null
};

__device__ __forceinline__ float gate_sigmoid(float x) { return 1.f / (1.f + __expf(-x)); }

template <int D, bool QF, bool FG>
__global__ __launch_bounds__(256, 2) void readout_kernel(
    const uint16_t *__restrict__ q, int64_t q_row, int64_t q_head, const float *__restrict__ prefix,
    const float *__restrict__ suffix, const float *__restrict__ logsum, const float *__restrict__ text,
    const int *__restrict__ bounds, int use_alpha, const uint16_t *__restrict__ norm_w, ReadoutGate gin,
    uint16_t *__restrict__ out, int64_t out_row, int F, int f0, int T, int heads) {
  constexpr int LP = D + 8, NS = D / 16, NO = D / 32, YP = D + 8, CPR = D / 8;  // CPR: 16-byte chunks per row
  constexpr int RPI = 64 / CPR;                                                  // rows per wave instruction
  __shared__ __attribute__((aligned(16))) uint16_t Ls[D * LP];
  __shared__ __attribute__((aligned(16))) uint16_t Ys[FG ? 1 : 4][FG ? 8 : 32 * YP];
  __shared__ __attribute__((aligned(16))) uint16_t Wg[FG ? D * LP : 8];
  __shared__ float Bg[FG ? D : 1];
  __shared__ float dec[2][D];
  __shared__ __attribute__((aligned(16))) uint16_t Wn[D];
  const int fh = blockIdx.x, fl = fh / heads, h = fh - fl * heads, f = f0 + fl;  // fl: frame within the range
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int lo = max(bounds[2 * f], 0), hi = min(bounds[2 * f + 1], F - 1);
  const bool has_b = lo - 1 >= 0, has_a = hi + 1 < F;
  const int bb = min(max(lo, 0), F), ba = min(max(hi + 1, 0), F);
  if (tid < D) {
    const int64_t hd = (int64_t)heads * D, e = (int64_t)h * D + tid;
    dec[0][tid] = use_alpha ? expf(logsum[(f + 1) * hd + e] - logsum[bb * hd + e]) : 1.f;
    dec[1][tid] = use_alpha ? expf(logsum[ba * hd + e] - logsum[f * hd + e]) : 1.f;
  }
  const float *before = has_b ? prefix + ((int64_t)(lo - 1) * heads + h) * D * D
                              : (text ? text + (int64_t)h * D * D : nullptr);
  const float *after = has_a ? suffix + ((int64_t)(hi + 1) * heads + h) * D * D
                             : (text ? text + (int64_t)h * D * D : nullptr);
  // the two states in halves, each half's loads issued before any of its use (D * D / 4
  // float4 per state, N4 per thread)
  constexpr int N4 = D * D / 4 / 256, H4 = N4 > 8 ? 8 : N4;
#pragma unroll
  for (int u0 = 0; u0 < N4; u0 += H4) {
    f32x4_t bv[H4], av[H4];
#pragma unroll
    for (int u = 0; u < H4; ++u) {
      const int i4 = tid + 256 * (u0 + u);
      bv[u] = before ? reinterpret_cast<const f32x4_t *>(before)[i4] : f32x4_t{0.f, 0.f, 0.f, 0.f};
      av[u] = after ? reinterpret_cast<const f32x4_t *>(after)[i4] : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    if (u0 == 0) __syncthreads();  // dec
#pragma unroll
    for (int u = 0; u < H4; ++u) {
      const int e0 = 4 * (tid + 256 * (u0 + u)), vv = e0 / D, kk = e0 - vv * D;
      float x[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        x[e] = __fadd_rn(before ? __fmul_rn(bv[u][e], dec[0][kk + e]) : 0.f,
                         after ? __fmul_rn(av[u][e], dec[1][kk + e]) : 0.f);
      *reinterpret_cast<u32x2_t *>(Ls + vv * LP + kk) = u32x2_t{pack_bf2(x[0], x[1]), pack_bf2(x[2], x[3])};
    }
  }
  if (tid < D / 4) *reinterpret_cast<u32x2_t *>(Wn + 4 * tid) = *reinterpret_cast<const u32x2_t *>(norm_w + 4 * tid);
  if constexpr (FG) {
#pragma unroll
    for (int u = 0; u < D * CPR / 256; ++u) {
      const int e = tid + 256 * u, r = e / CPR, c = e - r * CPR;
      st16(Wg + r * LP + 8 * c, ld16(gin.w_up + ((int64_t)h * D + r) * D + 8 * c));
    }
    if (tid < D) Bg[tid] = gin.b_up ? bf2f(gin.b_up[h * D + tid]) : 0.f;
  }
  __syncthreads();

  // gate hidden rows of a tile (FG): lane = token, like q
  auto h_ptr = [&](int tile) __device__ {
    const int64_t row = (int64_t)fl * T + min(tile * 32 + l32, T - 1);
    return gin.hidden + row * gin.hidden_row + 8 * g;
  };

  // q tiles: lane = token; the next tile's raw q is loaded after this tile's features
  const int ntiles = (T + 31) / 32;
  auto q_ptr = [&](int tile) __device__ {
    const int64_t row = (int64_t)fl * T + min(tile * 32 + l32, T - 1);
    return q + row * q_row + (int64_t)h * q_head + 8 * g;
  };
  u32x4_t raw[NS];
  if (wave < ntiles) {
    const uint16_t *qp = q_ptr(wave);
#pragma unroll
    for (int st = 0; st < NS; ++st) raw[st] = ld16(qp + 16 * st);
  }
  uint16_t *Yw = Ys[FG ? 0 : wave];
  const int orow = lane / CPR, ochunk = lane % CPR;  // row-major pass: row it * RPI + orow, chunk ochunk
  for (int tile = wave; tile < ntiles; tile += 4) {
    // this tile's gate rows, row-major (used at the end of the tile)
    u32x4_t gv[FG ? 1 : 32 / RPI];
    if constexpr (!FG) {
#pragma unroll
      for (int it = 0; it < 32 / RPI; ++it) {
        const int t = min(tile * 32 + it * RPI + orow, T - 1);
        gv[it] = ld16(gin.gate + ((int64_t)fl * T + t) * gin.gate_row + (int64_t)h * D + 8 * ochunk);
      }
    }

    bf16x8_t qf[NS];
    if (QF) {
#pragma unroll
      for (int st = 0; st < NS; ++st) qf[st] = as_bf16x8(raw[st]);
      if (tile + 4 < ntiles) {
        const uint16_t *qp = q_ptr(tile + 4);
#pragma unroll
        for (int st = 0; st < NS; ++st) raw[st] = ld16(qp + 16 * st);
      }
    } else {
      // SiLU(q) rounded to bf16 (the reference materialises it), packed in pairs; its L2 norm
      u32x4_t sq[NS];
      float sumsq = 0.f;
#pragma unroll
      for (int st = 0; st < NS; ++st)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float lo_ = silu_bf(bf_lo(raw[st][w])), hi_ = silu_bf(bf_hi(raw[st][w]));
          sumsq += lo_ * lo_;
          sumsq += hi_ * hi_;
          sq[st][w] = pack_bf2(lo_, hi_);
        }
      if (tile + 4 < ntiles) {
        const uint16_t *qp = q_ptr(tile + 4);
#pragma unroll
        for (int st = 0; st < NS; ++st) raw[st] = ld16(qp + 16 * st);
      }
      sumsq += __shfl_xor(sumsq, 32);
      const float nrm = fmaxf(round_bf(sqrtf(sumsq)), 1e-6f), rn = 1.f / nrm;
#pragma unroll
      for (int st = 0; st < NS; ++st)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          qf[st][2 * w] = __builtin_bit_cast(__bf16, f2bf(div_bf(bf_lo(sq[st][w]), nrm, rn)));
          qf[st][2 * w + 1] = __builtin_bit_cast(__bf16, f2bf(div_bf(bf_hi(sq[st][w]), nrm, rn)));
        }
    }
    f32x16_t acc[NO];
#pragma unroll
    for (int mb = 0; mb < NO; ++mb) {
      acc[mb] = f32x16_t{};
#pragma unroll
      for (int st = 0; st < NS; ++st)
        acc[mb] = mfma_bf16_32x32x16(as_bf16x8(ld16(Ls + (32 * mb + l32) * LP + 16 * st + 8 * g)), qf[st], acc[mb]);
    }
    // FG: this tile's gate hidden rows, loaded once q's fragments are dead (used after the norm)
    u32x4_t hraw[FG ? NS : 1];
    if constexpr (FG) {
      const uint16_t *hp = h_ptr(tile);
#pragma unroll
      for (int st = 0; st < NS; ++st) hraw[st] = ld16(hp + 16 * st);
    }
    float ss = 0.f;
#pragma unroll
    for (int mb = 0; mb < NO; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = acc[mb][r];
        const float rb = round_bf(e);
        acc[mb][r] = rb;
        ss += rb * rb;
      }
    ss += __shfl_xor(ss, 32);
    const float nv = sqrtf(ss);
    const float inv = round_bf(1.f / sqrtf(nv * nv / (float)D + 1e-6f));
    if constexpr (FG) {
      // per 32-row block of v: the gate's pre-activation, transposed like r (rows = v, lane =
      // token), then out = bf16(y * gate), y = bf16(bf16(r * inv) * w), four consecutive v per
      // 8-byte store
      const int t = tile * 32 + l32;
#pragma unroll
      for (int mb = 0; mb < NO; ++mb) {
        __builtin_amdgcn_sched_barrier(0);  // one block's W_up fragments live at a time
        f32x16_t gacc = {};
#pragma unroll
        for (int st = 0; st < NS; ++st)
          gacc = mfma_bf16_32x32x16(as_bf16x8(ld16(Wg + (32 * mb + l32) * LP + 16 * st + 8 * g)),
                                    as_bf16x8(hraw[st]), gacc);
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const int v0 = 32 * mb + 8 * i4 + 4 * g;
          const u32x2_t nw = *reinterpret_cast<const u32x2_t *>(Wn + v0);
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t ww = nw[e >> 1];
            const float y = round_bf(round_bf(acc[mb][4 * i4 + e] * inv) * ((e & 1) ? bf_hi(ww) : bf_lo(ww)));
            const float gt = round_bf(gate_sigmoid(round_bf(gacc[4 * i4 + e] + Bg[v0 + e])));
            o[e] = y * gt;
          }
          if (t < T)
            *reinterpret_cast<u32x2_t *>(out + ((int64_t)fl * T + t) * out_row + (int64_t)h * D + v0) =
                u32x2_t{pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3])};
        }
      }
      continue;
    }
    // y = bf16(bf16(r * inv) * w) into the stage, row = token l32
#pragma unroll
    for (int mb = 0; mb < NO; ++mb)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int v0 = 32 * mb + 8 * i4 + 4 * g;
        const u32x2_t nw = *reinterpret_cast<const u32x2_t *>(Wn + v0);
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t ww = nw[e >> 1];
          y[e] = round_bf(acc[mb][4 * i4 + e] * inv) * ((e & 1) ? bf_hi(ww) : bf_lo(ww));
        }
        *reinterpret_cast<u32x2_t *>(Yw + l32 * YP + v0) = u32x2_t{pack_bf2(y[0], y[1]), pack_bf2(y[2], y[3])};
      }
    asm volatile("" ::: "memory");  // LDS operations of one wavefront complete in order
    // out = y * gate, row-major 16-byte pieces
#pragma unroll
    for (int it = 0; it < 32 / RPI; ++it) {
      const int tt = it * RPI + orow, t = tile * 32 + tt;
      const u32x4_t yv = *reinterpret_cast<const u32x4_t *>(Yw + tt * YP + 8 * ochunk);
      if (t < T) {
        u32x4_t o;
#pragma unroll
        for (int w = 0; w < 4; ++w)
          o[w] = pack_bf2(bf_lo(yv[w]) * bf_lo(gv[it][w]), bf_hi(yv[w]) * bf_hi(gv[it][w]));
        *reinterpret_cast<u32x4_t *>(out + ((int64_t)fl * T + t) * out_row + (int64_t)h * D + 8 * ochunk) = o;
      }
    }
    asm volatile("" ::: "memory");
  }
}

template <bool FG>
int launch_readout(const uint16_t *q, int64_t q_row, int64_t q_head, int q_features, const float *prefix,
                   const float *suffix, const float *alpha_logsum, const float *text_state, const int32_t *bounds,
                   int use_alpha, const uint16_t *norm_w, const ReadoutGate &gin, uint16_t *out, int64_t out_row,
                   int frames, int first_frame, int frame_count, int tokens, int heads, int head_dim, hipStream_t s) {
  VDNH3_HOST_CHECK(q_features == 0 || q_features == 1, VDNH3_ERR_INVALID, "readout: q_features must be 0 or 1");
  VDNH3_HOST_CHECK(first_frame >= 0 && frame_count > 0 && first_frame <= frames - frame_count, VDNH3_ERR_INVALID,
                   "readout: frame range [%d, %d + %d) is not inside the %d frames", first_frame, first_frame,
                   frame_count, frames);
  const dim3 grid(frame_count * heads);
#define VDNH3_RO(D, QF)                                                                                          \
  if (head_dim == D && q_features == QF)                                                                         \
    hipLaunchKernelGGL((readout_kernel<D, QF, FG>), grid, dim3(256), 0, s, q, q_row, q_head, prefix, suffix,      \
                       alpha_logsum, text_state, bounds, use_alpha, norm_w, gin, out, out_row, frames, first_frame, \
                       tokens, heads);
  VDNH3_RO(128, 0)
  VDNH3_RO(128, 1)
  VDNH3_RO(64, 0)
  VDNH3_RO(64, 1)
#undef VDNH3_RO
  return check_launch("readout");
}

// ---------------------------------------------------------------------------------------
// frame means: grid (frames, hidden / 256), 256 threads = 32 column groups of 8 columns x 8
// token lanes; token lane l sums tokens l, l + 8, ... with 16-byte loads, the 8 partial sums
// of a column are added in LDS. hidden and the row stride are multiples of 8 (host check).
__global__ __launch_bounds__(256) void frame_mean_kernel(const uint16_t *__restrict__ x, int64_t x_row, int T,
                                                         int hidden, float *__restrict__ out) {
  __shared__ float part[8][257];
  const int f = blockIdx.x, tid = threadIdx.x, cg = tid & 31, tl = tid >> 5;
  const int col = blockIdx.y * 256 + cg * 8;
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (col < hidden) {
    const uint16_t *p = x + (int64_t)f * T * x_row + col;
    int t = tl;
    for (; t + 24 < T; t += 32) {
      u32x4_t r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) r[u] = ld16(p + (int64_t)(t + 8 * u) * x_row);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int j = 0; j < 8; ++j) s[j] += bf2f(uint16_t((j & 1) ? (r[u][j >> 1] >> 16) : (r[u][j >> 1] & 0xffffu)));
    }
    for (; t < T; t += 8) {
      const u32x4_t r = ld16(p + (int64_t)t * x_row);
#pragma unroll
      for (int j = 0; j < 8; ++j) s[j] += bf2f(uint16_t((j & 1) ? (r[j >> 1] >> 16) : (r[j >> 1] & 0xffffu)));
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) part[tl][cg * 8 + j] = s[j];
  __syncthreads();
  const int c = blockIdx.y * 256 + tid;
  if (c < hidden) {
    float v = 0.f;
#pragma unroll
    for (int l = 0; l < 8; ++l) v += part[l][tid];
    out[(int64_t)f * hidden + c] = v / (float)T;
  }
}

// out[m][n] = sum_k x[m][k] W[n][k] (+ bias[n]) in fp32 (the small alpha projections: few rows,
// K up to the hidden size), grid (N / 4, M / 8).
template <bool WBF16>
__global__ __launch_bounds__(256) void linear_f32_kernel(const float *__restrict__ x, int64_t x_row,
                                                         const void *__restrict__ w, int64_t w_row,
                                                         const float *__restrict__ bias, float *__restrict__ out,
                                                         int64_t out_row, int M, int N, int K) {
  // one workgroup per block of 8 rows x 4 columns; its 256 threads split K (thread t takes
  // k = t, t + 256, ...), each holding the 32 partial sums, then a tree over the threads in LDS
  constexpr int BM = 8, BN = 4;
  __shared__ float red[BM * BN][257];
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN, tid = threadIdx.x;
  const float *xr[BM];
#pragma unroll
  for (int i = 0; i < BM; ++i) xr[i] = x + (int64_t)min(m0 + i, M - 1) * x_row;
  int64_t wo[BN];
#pragma unroll
  for (int j = 0; j < BN; ++j) wo[j] = (int64_t)min(n0 + j, N - 1) * w_row;
  float acc[BM][BN] = {};
  for (int k = tid; k < K; k += 256) {
    float wk[BN], xk[BM];
#pragma unroll
    for (int j = 0; j < BN; ++j)
      wk[j] = WBF16 ? bf2f(static_cast<const uint16_t *>(w)[wo[j] + k]) : static_cast<const float *>(w)[wo[j] + k];
#pragma unroll
    for (int i = 0; i < BM; ++i) xk[i] = xr[i][k];
#pragma unroll
    for (int i = 0; i < BM; ++i)
#pragma unroll
      for (int j = 0; j < BN; ++j) acc[i][j] = fmaf(xk[i], wk[j], acc[i][j]);
  }
#pragma unroll
  for (int i = 0; i < BM; ++i)
#pragma unroll
    for (int j = 0; j < BN; ++j) red[i * BN + j][tid] = acc[i][j];
  __syncthreads();
  // 32 outputs x 256 partials: thread group of 8 per output sums 32 partials each, then 3 shuffles
  const int o = tid >> 3, part = tid & 7;
  float sum = 0.f;
#pragma unroll
  for (int u = 0; u < 32; ++u) sum += red[o][part * 32 + u];
  sum += __shfl_xor(sum, 1);
  sum += __shfl_xor(sum, 2);
  sum += __shfl_xor(sum, 4);
  const int m = m0 + o / BN, n = n0 + o % BN;
  if (part == 0 && m < M && n < N) out[(int64_t)m * out_row + n] = sum + (bias ? bias[n] : 0.f);
}

// short K: one wavefront per output column n, lanes striding K, eight rows of x at a time
template <bool WBF16>
__global__ __launch_bounds__(256) void linear_f32_cols_kernel(const float *__restrict__ x, int64_t x_row,
                                                         const void *__restrict__ w, int64_t w_row,
                                                         const float *__restrict__ bias, float *__restrict__ out,
                                                         int64_t out_row, int M, int N, int K) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (n >= N) return;  // the whole wavefront leaves; no workgroup barrier follows
  const float bn = bias ? bias[n] : 0.f;
  for (int m0 = 0; m0 < M; m0 += 8) {
    const float *xr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xr[i] = x + (int64_t)min(m0 + i, M - 1) * x_row;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int k = lane; k < K; k += 64) {
      const float wk = WBF16 ? bf2f(static_cast<const uint16_t *>(w)[(int64_t)n * w_row + k])
                             : static_cast<const float *>(w)[(int64_t)n * w_row + k];
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = fmaf(xr[i][k], wk, acc[i]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) acc[i] += __shfl_xor(acc[i], o);
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (m0 + i < M) out[(int64_t)(m0 + i) * out_row + n] = acc[i] + bn;
    }
  }
}

// alpha[f][h][d] = exp(-exp(a_log[h]) * softplus(delta[f][h*D + d]))  (torch softplus, threshold 20)
__global__ void alpha_decay_kernel(const float *__restrict__ delta, const float *__restrict__ a_log,
                                   float *__restrict__ alpha, int64_t n, int heads, int D) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  const int h = (int)((e / D) % heads);
  const float x = delta[e];
  const float sp = x > 20.f ? x : log1pf(expf(x));
  alpha[e] = expf(-expf(a_log[h]) * sp);
}

// Sana rule (vdn_h3/branch.py:163-177): Phi = alpha[i] * (I - A / T)[i][j], J = B / sqrt(T), each
// product and difference rounded to fp32 on its own like the reference's tensor ops (contraction
// into fused multiply-adds is off for this kernel), then J * j_scale (the text state's exact 1/2).
// Phi may be null (not needed).
__global__ void sana_factor_kernel(const float *__restrict__ A, const float *__restrict__ B,
                                   const float *__restrict__ alpha, float *__restrict__ Phi, float *__restrict__ J,
                                   float inv_t, float inv_sqrt_t, float j_scale, int64_t n, int D) {
#pragma clang fp contract(off)
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  if (Phi) {
    const int64_t mat = e / ((int64_t)D * D);
    const int i = (int)((e / D) % D), j = (int)(e % D);
    const float a = alpha ? alpha[mat * D + i] : 1.f;
    const float scaled = inv_t * A[e];
    const float diff = (i == j ? 1.f : 0.f) - scaled;
    Phi[e] = a * diff;
  }
  const float jb = inv_sqrt_t * B[e];
  J[e] = jb * j_scale;
}

__global__ void fill_rows_bf16_kernel(uint16_t *__restrict__ p, int64_t ld, int rows, int cols, uint16_t value) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)rows * cols) return;
  const int64_t r = e / cols, c = e - r * cols;
  p[r * ld + c] = value;
}

int check_dim(int head_dim) {
  VDNH3_HOST_CHECK(head_dim == 64 || head_dim == 128, VDNH3_ERR_INVALID,
                   "the delta-rule kernels support head_dim 64 or 128, got %d", head_dim);
  return VDNH3_OK;
}

}  // namespace
}  // namespace vdnh3

using vdnh3::check_dim;
using vdnh3::check_launch;
using vdnh3::set_error;

extern "C" int vdnh3_frame_stats(const uint16_t *k, int64_t k_row, int64_t k_head, const uint16_t *v,
                                 int64_t v_row, int64_t v_head, int features, const uint16_t *beta,
                                 int64_t beta_row, int frames, int tokens, int heads, int head_dim, float *A,
                                 float *B, void *stream) {
  int rc = check_dim(head_dim);
  if (rc) return rc;
  VDNH3_HOST_CHECK(k && v && beta && A && B && frames > 0 && tokens > 0 && heads > 0, VDNH3_ERR_INVALID,
                   "frame_stats: empty or null operand");
  VDNH3_HOST_CHECK(k_row % 8 == 0 && k_head % 8 == 0 && v_row % 8 == 0 && v_head % 8 == 0 &&
                       reinterpret_cast<uintptr_t>(k) % 16 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0,
                   VDNH3_ERR_INVALID, "frame_stats: k/v must be 16-byte aligned with strides multiple of 8");
  VDNH3_HOST_CHECK((features & ~7) == 0, VDNH3_ERR_INVALID, "frame_stats: unknown feature flags %d", features);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(frames * heads);
#define VDNH3_FS(D, KF, VF, AB)                                                                                \
  if (head_dim == D && (features & 1) == KF && ((features >> 1) & 1) == VF && ((features >> 2) & 1) == AB)   \
    hipLaunchKernelGGL((vdnh3::frame_stats_kernel<D, KF, VF, AB>), grid, dim3(256), 0, s, k, k_row, k_head, v, \
                       v_row, v_head, beta, beta_row, tokens, heads, A, B);
#define VDNH3_FS_D(D)    \
  VDNH3_FS(D, 0, 0, 0)   \
  VDNH3_FS(D, 1, 0, 0)   \
  VDNH3_FS(D, 0, 1, 0)   \
  VDNH3_FS(D, 1, 1, 0)   \
  VDNH3_FS(D, 0, 0, 1)   \
  VDNH3_FS(D, 1, 0, 1)   \
  VDNH3_FS(D, 0, 1, 1)   \
  VDNH3_FS(D, 1, 1, 1)
  VDNH3_FS_D(128)
  VDNH3_FS_D(64)
#undef VDNH3_FS_D
#undef VDNH3_FS
  return check_launch("frame_stats");
}

extern "C" int vdnh3_delta_factor(const float *A, const float *B, const float *alpha, float *phi, float *jay,
                                  float jay_scale, int32_t *info, int n, int head_dim, void *stream) {
  int rc = check_dim(head_dim);
  if (rc) return rc;
  VDNH3_HOST_CHECK(A && B && jay && info && n > 0, VDNH3_ERR_INVALID, "delta_factor: empty or null operand");
  VDNH3_HOST_CHECK(reinterpret_cast<uintptr_t>(B) % 16 == 0, VDNH3_ERR_INVALID, "delta_factor: B must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (head_dim == 128)
    hipLaunchKernelGGL(vdnh3::factor_kernel<128>, dim3(n), dim3(256), 0, s, A, B, alpha, phi, jay, jay_scale, info);
  else
    hipLaunchKernelGGL(vdnh3::factor_kernel<64>, dim3(n), dim3(256), 0, s, A, B, alpha, phi, jay, jay_scale, info);
  return check_launch("delta_factor");
}

extern "C" int vdnh3_sana_factor(const float *A, const float *B, const float *alpha, float *phi, float *jay,
                                 float jay_scale, int tokens_per_frame, int n, int head_dim, void *stream) {
  VDNH3_HOST_CHECK(A && B && jay && n > 0 && head_dim > 0 && tokens_per_frame > 0, VDNH3_ERR_INVALID,
                   "sana_factor: empty or null operand");
  const int64_t total = (int64_t)n * head_dim * head_dim;
  // the reference's Python floats 1 / T and (1 / T) ** 0.5, rounded once to fp32
  const double inv_t = 1.0 / (double)tokens_per_frame;
  hipLaunchKernelGGL(vdnh3::sana_factor_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), A, B, alpha, phi, jay, (float)inv_t, (float)sqrt(inv_t),
                     jay_scale, total, head_dim);
  return check_launch("sana_factor");
}

extern "C" int vdnh3_delta_scan(const float *phi, const float *jay, const float *init, float *prefix, float *suffix,
                                int frames, int heads, int head_dim, void *stream) {
  int rc = check_dim(head_dim);
  if (rc) return rc;
  VDNH3_HOST_CHECK(phi && jay && prefix && suffix && frames > 0 && heads > 0, VDNH3_ERR_INVALID,
                   "delta_scan: empty or null operand");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(heads * 2 * (head_dim / 32));
  if (head_dim == 128)
    hipLaunchKernelGGL(vdnh3::scan_kernel<128>, grid, dim3(256), 0, s, phi, jay, init, prefix, suffix, frames, heads);
  else
    hipLaunchKernelGGL(vdnh3::scan_kernel<64>, grid, dim3(128), 0, s, phi, jay, init, prefix, suffix, frames, heads);
  return check_launch("delta_scan");
}

extern "C" int vdnh3_alpha_logsum(const float *alpha, int frames, int heads, int head_dim, float *out, void *stream) {
  VDNH3_HOST_CHECK(alpha && out && frames > 0 && heads > 0 && head_dim > 0, VDNH3_ERR_INVALID,
                   "alpha_logsum: empty or null operand");
  const int hd = heads * head_dim;
  hipLaunchKernelGGL(vdnh3::alpha_logsum_kernel, dim3((hd + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                     alpha, out, frames, hd);
  return check_launch("alpha_logsum");
}

extern "C" int vdnh3_readout(const uint16_t *q, int64_t q_row, int64_t q_head, int q_features,
                             const float *prefix, const float *suffix, const float *alpha_logsum,
                             const float *text_state, const int32_t *bounds, int use_alpha, const uint16_t *norm_w,
                             const uint16_t *gate, int64_t gate_row, uint16_t *out, int64_t out_row, int frames,
                             int first_frame, int frame_count, int tokens, int heads, int head_dim, void *stream) {
  int rc = check_dim(head_dim);
  if (rc) return rc;
  VDNH3_HOST_CHECK(q && prefix && suffix && (alpha_logsum || !use_alpha) && bounds && norm_w && gate && out &&
                       frames > 0 && tokens > 0,
                   VDNH3_ERR_INVALID, "readout: empty or null operand");
  VDNH3_HOST_CHECK(q_row % 8 == 0 && q_head % 8 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                       gate_row % 8 == 0 && out_row % 8 == 0 && reinterpret_cast<uintptr_t>(gate) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(out) % 16 == 0 && reinterpret_cast<uintptr_t>(norm_w) % 8 == 0 &&
                       reinterpret_cast<uintptr_t>(prefix) % 16 == 0 && reinterpret_cast<uintptr_t>(suffix) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(text_state) % 16 == 0,
                   VDNH3_ERR_INVALID, "readout: misaligned q / gate / out / norm weight / states");
  const vdnh3::ReadoutGate gin{gate, gate_row, nullptr, 0, nullptr, nullptr};
  return vdnh3::launch_readout<false>(q, q_row, q_head, q_features, prefix, suffix, alpha_logsum, text_state, bounds,
                                      use_alpha, norm_w, gin, out, out_row, frames, first_frame, frame_count, tokens,
                                      heads, head_dim, static_cast<hipStream_t>(stream));
}

extern "C" int vdnh3_readout_fused_gate(const uint16_t *q, int64_t q_row, int64_t q_head, int q_features,
                                        const float *prefix, const float *suffix, const float *alpha_logsum,
                                        const float *text_state, const int32_t *bounds, int use_alpha,
                                        const uint16_t *norm_w, const uint16_t *gate_hidden, int64_t hidden_row,
                                        const uint16_t *gate_up_w, const uint16_t *gate_up_b, uint16_t *out,
                                        int64_t out_row, int frames, int first_frame, int frame_count, int tokens,
                                        int heads, int head_dim, void *stream) {
  int rc = check_dim(head_dim);
  if (rc) return rc;
  VDNH3_HOST_CHECK(q && prefix && suffix && (alpha_logsum || !use_alpha) && bounds && norm_w && gate_hidden &&
                       gate_up_w && out && frames > 0 && tokens > 0,
                   VDNH3_ERR_INVALID, "readout: empty or null operand");
  VDNH3_HOST_CHECK(q_row % 8 == 0 && q_head % 8 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                       hidden_row % 8 == 0 && reinterpret_cast<uintptr_t>(gate_hidden) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(gate_up_w) % 16 == 0 && out_row % 4 == 0 &&
                       reinterpret_cast<uintptr_t>(out) % 8 == 0 && reinterpret_cast<uintptr_t>(norm_w) % 8 == 0 &&
                       reinterpret_cast<uintptr_t>(prefix) % 16 == 0 && reinterpret_cast<uintptr_t>(suffix) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(text_state) % 16 == 0,
                   VDNH3_ERR_INVALID, "readout: misaligned q / gate hidden / gate weight / out / norm weight / states");
  const vdnh3::ReadoutGate gin{nullptr, 0, gate_hidden, hidden_row, gate_up_w, gate_up_b};
  return vdnh3::launch_readout<true>(q, q_row, q_head, q_features, prefix, suffix, alpha_logsum, text_state, bounds,
                                     use_alpha, norm_w, gin, out, out_row, frames, first_frame, frame_count, tokens,
                                     heads, head_dim, static_cast<hipStream_t>(stream));
}

extern "C" int vdnh3_frame_mean(const uint16_t *x, int64_t x_row, int frames, int tokens, int hidden, float *out,
                                void *stream) {
  VDNH3_HOST_CHECK(x && out && frames > 0 && tokens > 0 && hidden > 0, VDNH3_ERR_INVALID,
                   "frame_mean: empty or null operand");
  VDNH3_HOST_CHECK(hidden % 8 == 0 && x_row % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0, VDNH3_ERR_INVALID,
                   "frame_mean: hidden and the row stride must be multiples of 8, x 16-byte aligned");
  hipLaunchKernelGGL(vdnh3::frame_mean_kernel, dim3(frames, (hidden + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, x_row, tokens, hidden, out);
  return check_launch("frame_mean");
}

extern "C" int vdnh3_linear_f32(const float *x, int64_t x_row, const void *w, int w_bf16, int64_t w_row,
                                const float *bias, float *out, int64_t out_row, int M, int N, int K, void *stream) {
  VDNH3_HOST_CHECK(x && w && out && M > 0 && N > 0 && K > 0, VDNH3_ERR_INVALID, "linear_f32: empty or null operand");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (K >= 1024) {  // long K: split over the workgroup's threads
    const dim3 grid((unsigned)((N + 3) / 4), (unsigned)((M + 7) / 8));
    if (w_bf16)
      hipLaunchKernelGGL(vdnh3::linear_f32_kernel<true>, grid, dim3(256), 0, s, x, x_row, w, w_row, bias, out,
                         out_row, M, N, K);
    else
      hipLaunchKernelGGL(vdnh3::linear_f32_kernel<false>, grid, dim3(256), 0, s, x, x_row, w, w_row, bias, out,
                         out_row, M, N, K);
  } else {
    const dim3 grid((unsigned)((N + 3) / 4));
    if (w_bf16)
      hipLaunchKernelGGL(vdnh3::linear_f32_cols_kernel<true>, grid, dim3(256), 0, s, x, x_row, w, w_row, bias, out,
                         out_row, M, N, K);
    else
      hipLaunchKernelGGL(vdnh3::linear_f32_cols_kernel<false>, grid, dim3(256), 0, s, x, x_row, w, w_row, bias, out,
                         out_row, M, N, K);
  }
  return check_launch("linear_f32");
}

extern "C" int vdnh3_alpha_decay(const float *delta, const float *a_log, float *alpha, int frames, int heads,
                                 int head_dim, void *stream) {
  VDNH3_HOST_CHECK(delta && a_log && alpha && frames > 0 && heads > 0 && head_dim > 0, VDNH3_ERR_INVALID,
                   "alpha_decay: empty or null operand");
  const int64_t n = (int64_t)frames * heads * head_dim;
  hipLaunchKernelGGL(vdnh3::alpha_decay_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), delta, a_log, alpha, n, heads, head_dim);
  return check_launch("alpha_decay");
}

extern "C" int vdnh3_fill_rows_bf16(uint16_t *p, int64_t ld, int rows, int cols, float value, void *stream) {
  VDNH3_HOST_CHECK(p && rows >= 0 && cols >= 0 && ld >= cols, VDNH3_ERR_INVALID, "fill_rows: bad operand");
  if (rows == 0 || cols == 0) return VDNH3_OK;
  const int64_t n = (int64_t)rows * cols;
  const uint32_t u = __builtin_bit_cast(uint32_t, value);
  const uint16_t b = uint16_t((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  hipLaunchKernelGGL(vdnh3::fill_rows_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), p, ld, rows, cols, b);
  return check_launch("fill_rows_bf16");
}
