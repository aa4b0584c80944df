// Token-level chunked Gated DeltaNet on gfx950: the chunk-64 gated delta rule
//   S_t = a_t S_{t-1} (I - b_t k_t k_t^T) + b_t v_t k_t^T,   o_t = S_t q_t,   a_t = exp(g_t)
// per head, S (dv x dk) in fp32. This path is not part of hyukudan/ComfyUI-Kirei-VDN-H3, whose
// Video Delta Attention solves its delta rule per frame (vdn_h3/branch.py:148-160); it is the
// published Gated DeltaNet (Yang, Kautz, Hatamizadeh 2024) in its chunk (WY) form. With the
// in-chunk cumulative log-decay G_t and chunk length C = 64:
//   A[t][j] = b_t exp(G_t - G_j) k_t.k_j (j < t),   (I + A) W = diag(b e^G) K,   (I + A) U~ = diag(b) V
//   U = U~ - W S0^T,   O = diag(e^G) Q S0^T + (Q K^T o D) U,   D[t][j] = exp(G_t - G_j) (j <= t)
//   S_C = e^{G_C} S0 + U^T diag(e^{G_C - G}) K
//
// gdn_prep_kernel (grid heads x chunks, fully parallel): K K^T and Q K^T on bf16 MFMA; the
// inverse T = (I + A)^-1 in fp32 by 16 x 16 blocks, then W = T diag(b e^G) K and U~ = T diag(b) V
// on bf16 MFMA (T's scaled columns rounded to bf16); writes W, U~, Q^ = e^G Q,
// K^ = e^{G_C - G} K, P = Q K^T o D (bf16, each in the fragment order of the scan wavefront
// that reads it) and G (fp32) for each chunk, as 16-byte stores. When the host pipelines the
// segments of a call (two streams), the prep of the next segment runs beside the scan, whose four workgroups per head share each chunk's W, Q^, K^ and P
// through L2; the prep's q / k / v reads and its workspace writes carry the non-temporal hint,
// so that they stream past L2 instead of displacing those lines (3% faster).
// gdn_scan_kernel (grid heads x dv/32, sequential over chunks): one workgroup carries a 32-row
// slice of the state in MFMA accumulators (fp32); per chunk U = U~ - W S^T, O = Q^ S^T + P U and
// S = e^{G_C} S + U^T K^, each wavefront loading its operands into registers two chunks ahead.
#include "common.h"

namespace vdnh3 {
namespace {

constexpr int kGdnC = 64;  // chunk length

template <int D>
struct GdnWs {  // per (chunk, head) workspace element counts
  static constexpr int64_t W = (int64_t)kGdnC * D, U = W, Q = W, K = W, P = (int64_t)kGdnC * kGdnC, G = kGdnC;
};

// The workspace holds each block in the fragment order of the scan wavefront that reads it, so
// that a wavefront's 16-byte fragment pieces lie in lane order (1 KB per load instruction). Scan
// wavefront w forms U and O for tokens 16 w .. 16 w + 15 on 16x16x32 MFMAs and carries the state
// block of dk columns 32 w .. 32 w + 31 on 32x32x16 MFMAs:
//  - W, Q^ (128 columns: 4 k-steps of 32) and P (64 columns: 2 k-steps), A operands: piece
//    p = (w steps + s) 64 + lane holds row 16 w + lane % 16, columns 32 s + 8 (lane / 16) .. + 7;
//  - K^ = e^{G_C - G} K, B operand of state block w: piece (w 4 + s) 64 + lane holds tokens
//    16 s + 8 (lane / 32) .. + 7 of column 32 w + lane % 32;
//  - U~ for state slice sl in the 16x16 accumulator layout: piece (sl 4 + w) 64 + lane holds, at
//    element 4 nb + i, row 16 w + 4 (lane / 16) + i of column 32 sl + 16 nb + lane % 16.
__device__ __forceinline__ int gdn_a_row(int p, int steps) { return 16 * (p / (64 * steps)) + (p & 15); }
__device__ __forceinline__ int gdn_a_col(int p, int steps) { return 32 * ((p >> 6) % steps) + 8 * ((p >> 4) & 3); }

template <int D>
__global__ __launch_bounds__(256) void gdn_prep_kernel(
    const uint16_t *__restrict__ q, int64_t q_row, int64_t q_head, const uint16_t *__restrict__ k, int64_t k_row,
    int64_t k_head, const uint16_t *__restrict__ v, int64_t v_row, int64_t v_head, const float *__restrict__ beta,
    int64_t b_row, const float *__restrict__ lg, int64_t g_row, int T, int heads, uint16_t *__restrict__ Wo,
    uint16_t *__restrict__ Uo, uint16_t *__restrict__ Qo, uint16_t *__restrict__ Ko, uint16_t *__restrict__ Po,
    float *__restrict__ Go) {
  constexpr int C = kGdnC, KP = D + 8, CH = D / 8, AP = C + 4, PP = C + 8;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[C * KP], Qs[C * KP], Vs[C * KP], Ps[C * PP];
  __shared__ __attribute__((aligned(16))) float As[C * AP];  // rows 16-byte aligned: vector reads in the solve
  __shared__ float Gs[C], Bs[C], Eg[C], Ec[C];                // G, b, e^G, e^{G_C - G}
  const int h = blockIdx.x, c = blockIdx.y, t0 = c * C, n = min(C, T - t0);  // heads fastest: rows read whole
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, gl = lane >> 5;
  const int64_t ch = (int64_t)c * heads + h;

  // rows of the chunk (tokens past T are zero: they add nothing and keep the decay)
  for (int e = tid; e < C * CH; e += 256) {
    const int r = e / CH, cc = e - r * CH;
    u32x4_t kv = {0, 0, 0, 0}, qv = kv, vv = kv;
    if (r < n) {
      const int64_t row = t0 + r;
      kv = ld16_stream(k + row * k_row + (int64_t)h * k_head + 8 * cc);
      qv = ld16_stream(q + row * q_row + (int64_t)h * q_head + 8 * cc);
      vv = ld16_stream(v + row * v_row + (int64_t)h * v_head + 8 * cc);
    }
    st16(Ks + r * KP + 8 * cc, kv);
    st16(Qs + r * KP + 8 * cc, qv);
    st16(Vs + r * KP + 8 * cc, vv);
  }
  if (wave == 0) {  // inclusive prefix sum of the log-decay over the chunk, and its exponentials
    float x = lane < n ? lg[(int64_t)(t0 + lane) * g_row + h] : 0.f;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float y = __shfl_up(x, o);
      if (lane >= o) x += y;
    }
    Gs[lane] = x;
    Bs[lane] = lane < n ? beta[(int64_t)(t0 + lane) * b_row + h] : 0.f;
    Eg[lane] = expf(x);
    Ec[lane] = expf(__shfl(x, 63) - x);
  }
  __syncthreads();

  // K K^T and Q K^T: wave w owns the 32 x 32 block (w / 2, w % 2); A (fp32) and P (bf16) to LDS
  {
    const int mb = wave >> 1, nb = wave & 1;
    f32x16_t akk = {}, aqk = {};
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      const bf16x8_t ak = as_bf16x8(ld16(Ks + (32 * mb + l32) * KP + 16 * s + 8 * gl));
      const bf16x8_t aq = as_bf16x8(ld16(Qs + (32 * mb + l32) * KP + 16 * s + 8 * gl));
      const bf16x8_t bk = as_bf16x8(ld16(Ks + (32 * nb + l32) * KP + 16 * s + 8 * gl));
      akk = mfma_bf16_32x32x16(ak, bk, akk);
      aqk = mfma_bf16_32x32x16(aq, bk, aqk);
    }
    const int nn = 32 * nb + l32;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int m = 32 * mb + 8 * (i >> 2) + 4 * gl + (i & 3);
      const float dec = nn <= m ? expf(Gs[m] - Gs[nn]) : 0.f;
      As[m * AP + nn] = nn < m ? Bs[m] * dec * akk[i] : 0.f;
      Ps[m * PP + nn] = f2bf(aqk[i] * dec);
    }
  }
  __syncthreads();

  // Q^ = e^G Q, K^ = e^{G_C - G} K and P in the scan's fragment order (gdn_a_row): 16-byte
  // stores in piece order, before the solve overwrites Ks
  {
    uint16_t *qc = Qo + ch * GdnWs<D>::Q, *kc = Ko + ch * GdnWs<D>::K, *pc = Po + ch * GdnWs<D>::P;
#pragma unroll
    for (int u = 0; u < C * CH / 256; ++u) {
      const int p = tid + 256 * u, r = gdn_a_row(p, D / 32), k0 = gdn_a_col(p, D / 32);
      const u32x4_t x = ld16(Qs + r * KP + k0);
      const float sc = Eg[r];
      st16_stream(qc + 8 * p,
                  u32x4_t{pack_bf2(bf2f((uint16_t)x[0]) * sc, bf2f((uint16_t)(x[0] >> 16)) * sc),
                          pack_bf2(bf2f((uint16_t)x[1]) * sc, bf2f((uint16_t)(x[1] >> 16)) * sc),
                          pack_bf2(bf2f((uint16_t)x[2]) * sc, bf2f((uint16_t)(x[2] >> 16)) * sc),
                          pack_bf2(bf2f((uint16_t)x[3]) * sc, bf2f((uint16_t)(x[3] >> 16)) * sc)});
    }
#pragma unroll
    for (int u = 0; u < D * (C / 8) / 256; ++u) {
      const int e = tid + 256 * u, tc = e / D, d = e - tc * D;  // lanes walk d: conflict-free LDS reads
      float y[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = bf2f(Ks[(8 * tc + j) * KP + d]) * Ec[8 * tc + j];
      // K^ as the B operand of wave d / 32: piece (d / 32, tc / 2, lane 32 (tc & 1) + d % 32)
      st16_stream(kc + 8 * ((((d >> 5) * 4 + (tc >> 1)) << 6) + 32 * (tc & 1) + (d & 31)),
                  u32x4_t{pack_bf2(y[0], y[1]), pack_bf2(y[2], y[3]), pack_bf2(y[4], y[5]), pack_bf2(y[6], y[7])});
    }
#pragma unroll
    for (int u = 0; u < C * (C / 8) / 256; ++u) {
      const int p = tid + 256 * u, r = gdn_a_row(p, C / 32), j0 = gdn_a_col(p, C / 32);
      st16_stream(pc + 8 * p, ld16(Ps + r * PP + j0));
    }
    if (tid < C) Go[ch * GdnWs<D>::G + tid] = Gs[tid];
  }
  __syncthreads();

  // T = (I + A)^-1 (unit lower triangular) by 16 x 16 blocks, in fp32. T[i][j] (block of i at or
  // below the block of j) is kept transposed in As at As[j][i]: the blocks below the diagonal in
  // the upper triangle, the diagonal blocks whole (unit diagonal, zeros above it) in place of A's
  // diagonal blocks, which only their own solve reads. The diagonal blocks come from forward
  // substitution (wave I, lane c: column c of block I, stored as row 16 I + c of As); the blocks
  // below follow by distance d = I - J from the diagonal:
  //   X = sum_{K=J}^{I-1} A_IK T_KJ,   T_IJ = -T_II X
  // so X[r][c] is the dot product of As rows 16 I + r (A) and 16 J + c (T^T) over columns
  // 16 J .. 16 I - 1, and X sits in the (now free) Q staging area. Every load is unconditional:
  // no branch keeps the compiler from issuing them early.
  auto t_at = [&](int i, int j) __device__ { return As[j * AP + i]; };  // T[i][j], block(i) >= block(j)
  if (lane < 16) {
    const int I = wave, cc = lane;
    float t[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float acc = 0.f;
#pragma unroll
      for (int m = 0; m < r; ++m) acc = fmaf(As[(16 * I + r) * AP + 16 * I + m], t[m], acc);
      t[r] = r == cc ? 1.f : (r < cc ? 0.f : -acc);
    }
    // after every read of the block (program order within the wave)
    f32x4_t *row = reinterpret_cast<f32x4_t *>(As + (16 * I + cc) * AP + 16 * I);
#pragma unroll
    for (int q = 0; q < 4; ++q) row[q] = f32x4_t{t[4 * q], t[4 * q + 1], t[4 * q + 2], t[4 * q + 3]};
  }
  float *Xs = reinterpret_cast<float *>(Qs);  // [block][16][16]
  const int br = tid >> 4, bc = tid & 15;     // this thread's element of every 16 x 16 block
#pragma unroll
  for (int d = 1; d < 4; ++d) {
    __syncthreads();
#pragma unroll
    for (int b = 0; b < 4 - d; ++b) {
      const int I = d + b, J = b;
      const f32x4_t *ra = reinterpret_cast<const f32x4_t *>(As + (16 * I + br) * AP + 16 * J);
      const f32x4_t *rt = reinterpret_cast<const f32x4_t *>(As + (16 * J + bc) * AP + 16 * J);
      float x = 0.f;
#pragma unroll
      for (int q = 0; q < 4 * d; ++q) {
        const f32x4_t a4 = ra[q], t4 = rt[q];
        x = fmaf(a4[0], t4[0], x);
        x = fmaf(a4[1], t4[1], x);
        x = fmaf(a4[2], t4[2], x);
        x = fmaf(a4[3], t4[3], x);
      }
      Xs[(b * 16 + br) * 16 + bc] = x;
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < 4 - d; ++b) {
      const int I = d + b, J = b;
      float y = Xs[(b * 16 + br) * 16 + bc];
#pragma unroll
      for (int m = 0; m < 15; ++m) {
        const float tm = t_at(16 * I + br, 16 * I + m);  // T_II[br][m], the unit diagonal left out
        y = fmaf(m < br ? tm : 0.f, Xs[(b * 16 + m) * 16 + bc], y);
      }
      As[(16 * J + bc) * AP + 16 * I + br] = -y;
    }
  }
  __syncthreads();

  // Tw = T diag(b e^G), Tu = T diag(b) in bf16, row-major 64 x 64 with 16-byte chunk c of row i at
  // c ^ ((i >> 1) & 7), in the Q staging area (free now)
  uint16_t *Tw = Qs, *Tu = Qs + C * C;
#pragma unroll
  for (int u = 0; u < C * (C / 8) / 256; ++u) {
    const int e = tid + 256 * u, i = e & 63, jc = e >> 6;  // lanes walk rows: conflict-free reads
    float w[8], v8[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int j = 8 * jc + jj;
      const float ta = t_at(i, j);  // A[j][i] when block(j) > block(i): read always, then dropped
      const float tv = (j >> 4) > (i >> 4) ? 0.f : ta;
      v8[jj] = tv * Bs[j];
      w[jj] = v8[jj] * Eg[j];
    }
    const int off = i * C + 8 * (jc ^ ((i >> 1) & 7));
    st16(Tw + off, u32x4_t{pack_bf2(w[0], w[1]), pack_bf2(w[2], w[3]), pack_bf2(w[4], w[5]), pack_bf2(w[6], w[7])});
    st16(Tu + off,
         u32x4_t{pack_bf2(v8[0], v8[1]), pack_bf2(v8[2], v8[3]), pack_bf2(v8[4], v8[5]), pack_bf2(v8[6], v8[7])});
  }
  __syncthreads();

  // W = Tw K and U~ = Tu V on MFMA: wave w owns columns 32 w .. 32 w + 31 of both, all 64 rows.
  // B fragments are 8 tokens of one column (8 LDS reads); row block 0 skips tokens 32..63 (zero in Tw, Tu).
  {
    f32x16_t aw[2] = {}, au[2] = {};
#pragma unroll
    for (int s = 0; s < C / 16; ++s) {
      bf16x8_t bk, bv;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int j = 16 * s + 8 * gl + jj;
        bk[jj] = __builtin_bit_cast(__bf16, Ks[j * KP + 32 * wave + l32]);
        bv[jj] = __builtin_bit_cast(__bf16, Vs[j * KP + 32 * wave + l32]);
      }
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        if (mb == 0 && s >= 2) continue;
        const int i = 32 * mb + l32, off = i * C + 8 * ((2 * s + gl) ^ ((i >> 1) & 7));
        aw[mb] = mfma_bf16_32x32x16(as_bf16x8(ld16(Tw + off)), bk, aw[mb]);
        au[mb] = mfma_bf16_32x32x16(as_bf16x8(ld16(Tu + off)), bv, au[mb]);
      }
    }
    __syncthreads();  // every read of Ks / Vs is done: W and U~ replace them
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = 32 * mb + 8 * (i >> 2) + 4 * gl + (i & 3);
        Ks[r * KP + 32 * wave + l32] = f2bf(aw[mb][i]);
        Vs[r * KP + 32 * wave + l32] = f2bf(au[mb][i]);
      }
  }
  __syncthreads();
  {
    uint16_t *wc = Wo + ch * GdnWs<D>::W, *uc = Uo + ch * GdnWs<D>::U;
#pragma unroll
    for (int u = 0; u < C * CH / 256; ++u) {
      const int p = tid + 256 * u;
      st16_stream(wc + 8 * p, ld16(Ks + gdn_a_row(p, D / 32) * KP + gdn_a_col(p, D / 32)));
      // U~ piece p = (sl 4 + w) 64 + L: column 32 sl + 16 nb + L % 16 at rows 16 w + 4 (L / 16) + i
      const int L = p & 63, r0 = 16 * ((p >> 6) & 3) + 4 * (L >> 4), c0 = 32 * (p >> 8) + (L & 15);
      uint16_t e[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) e[x] = Vs[(r0 + (x & 3)) * KP + c0 + 16 * (x >> 2)];
      st16_stream(uc + 8 * p, u32x4_t{e[0] | (uint32_t)e[1] << 16, e[2] | (uint32_t)e[3] << 16,
                                      e[4] | (uint32_t)e[5] << 16, e[6] | (uint32_t)e[7] << 16});
    }
  }
}

// One workgroup = head h, state rows (dv) 32 sl .. 32 sl + 31, four wavefronts alike: wave w forms
// tokens 16 w .. 16 w + 15 of U = U~ - W S^T and of O = Q^ S^T + P U on 16x16x32 MFMAs, and
// carries the state block of dk columns 32 w .. 32 w + 31 as one 32x32 MFMA accumulator (fp32),
// S = e^{G_C} S + U^T K^. s_init and s_final may be the same buffer: a workgroup reads its slice
// of s_init before anything else and writes the same slice of s_final last.
//
// Every wavefront reads only its own part of a chunk's operands (its 16 rows of W, Q^, P and U~,
// its K^ block), stored in its fragment order, so each wavefront loads them straight into
// registers (1 KB per load instruction), two chunks ahead: a ring of three register sets, which
// keeps two chunks' loads in flight behind the step that computes. The state's bf16 copy (Sb) and
// U (Ut, transposed) are exchanged through LDS; the outputs of chunk c go to LDS (Os) in step c
// and to global memory at the start of step c + 1 (one 16-byte store per thread).
template <int D>
__global__ __launch_bounds__(256) void gdn_scan_kernel(
    const u32x4_t *__restrict__ Wi, const u32x4_t *__restrict__ Ui, const u32x4_t *__restrict__ Qi,
    const u32x4_t *__restrict__ Ki, const u32x4_t *__restrict__ Pi, const float *__restrict__ Gi, int n_chunks,
    int T, int heads, const float *s_init, float *s_final, uint16_t *__restrict__ out,
    int64_t o_row, int64_t o_head) {
  static_assert(D == 128, "the scan keeps one 32-column state block per wave: head_dim 128");
  constexpr int C = kGdnC, KP = D + 8, CP = C + 8, OP = 32 + 8;
  // Ut and Os hold two chunks each: P U of chunk c and its outputs are finished in step c + 1
  __shared__ __attribute__((aligned(16))) uint16_t Sb[32 * KP], Ut[2][32 * CP], Os[2][C * OP];
  const int h = blockIdx.x, sl = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, gl = lane >> 5;  // 32x32 fragment coordinates
  const int l16 = lane & 15, g4 = lane >> 4;  // 16x16 fragment coordinates

  // one chunk's operands of this wavefront; g = G of lane (a vector load, so its wait is a vmcnt)
  struct Frags {
    u32x4_t w[D / 32], q[D / 32], p[C / 32], u, k[C / 16];
    float g;
  };
  const u32x4_t *w_src = Wi + (wave * (D / 32) << 6) + lane, *q_src = Qi + (wave * (D / 32) << 6) + lane;
  const u32x4_t *p_src = Pi + (wave * (C / 32) << 6) + lane, *u_src = Ui + ((sl * 4 + wave) << 6) + lane;
  const u32x4_t *k_src = Ki + (wave * (C / 16) << 6) + lane;
  auto load = [&](int c, Frags &f) __device__ {
    c = c < n_chunks ? c : n_chunks - 1;  // past the end: the last chunk again, never used
    const int64_t ch = (int64_t)c * heads + h;
    const int64_t o16 = ch * (GdnWs<D>::W / 8), p16 = ch * (GdnWs<D>::P / 8);  // 16-byte pieces
#pragma unroll
    for (int s = 0; s < D / 32; ++s) f.w[s] = w_src[o16 + 64 * s];
#pragma unroll
    for (int s = 0; s < D / 32; ++s) f.q[s] = q_src[o16 + 64 * s];
#pragma unroll
    for (int s = 0; s < C / 32; ++s) f.p[s] = p_src[p16 + 64 * s];
    f.u = u_src[o16];
#pragma unroll
    for (int s = 0; s < C / 16; ++s) f.k[s] = k_src[o16 + 64 * s];
    f.g = Gi[ch * GdnWs<D>::G + lane];
  };

  // state block of this wave: S[v = 32 sl + row][k = 32 wave + l32]
  f32x16_t st = {};
  if (s_init) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int vr = 8 * (i >> 2) + 4 * gl + (i & 3);
      st[i] = s_init[((int64_t)h * D + 32 * sl + vr) * D + 32 * wave + l32];
    }
  }
  auto write_sb = [&]() __device__ {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int vr = 8 * (i >> 2) + 4 * gl + (i & 3);
      Sb[vr * KP + 32 * wave + l32] = f2bf(st[i]);
    }
  };
  // this wave's LDS writes are done, then the barrier
  auto lds_barrier = [&]() __device__ {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    bare_barrier();
  };
  // outputs of chunk c (in Os[c & 1]) to global memory: thread = (token tid / 4, 8 dv columns)
  auto store_o = [&](int c) __device__ {
    const int tk = tid >> 2, pc = tid & 3, tok = c * C + tk;
    const u32x4_t val = ld16(Os[c & 1] + tk * OP + 8 * pc);
    if (tok < T) st16(out + (int64_t)tok * o_row + (int64_t)h * o_head + 32 * sl + 8 * pc, val);
  };

  // O of chunk c - 1 between its two halves: Q^ S^T (step c - 1), P U (step c)
  f32x4_t oprev[2] = {};
  // P U of the chunk whose P fragments are p and whose U is in Ut[b], onto oprev
  auto pu = [&](const u32x4_t (&p)[C / 32], int b) __device__ {
#pragma unroll
    for (int s = 0; s < C / 32; ++s)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        oprev[nb] = mfma_bf16_16x16x32(as_bf16x8(p[s]),
                                       as_bf16x8(ld16(Ut[b] + (16 * nb + l16) * CP + 32 * s + 8 * g4)), oprev[nb]);
  };
  auto write_o = [&](int b) __device__ {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) Os[b][(16 * wave + 4 * g4 + i) * OP + 16 * nb + l16] = f2bf(oprev[nb][i]);
  };

  // Step c computes chunk c from register set f; `ahead` holds chunk c - 1 until it is reloaded
  // with chunk c + 2. The U chain (W S^T, U, Ut, the state update, Sb) is the critical path, so
  // its MFMAs issue first; O's products follow it in the MFMA pipe and O of chunk c - 1 is
  // completed and written here, off that chain.
  auto step = [&](int c, const Frags &f, Frags &ahead) __device__ {
    const int b = c & 1;
    if (c > 1) store_o(c - 2);
    // (a) tokens 16 w .. 16 w + 15, state rows 16 nb .. 16 nb + 15: U = U~ - W S^T (S^T from Sb)
    f32x4_t ua[2] = {}, ocur[2] = {};
#pragma unroll
    for (int s = 0; s < D / 32; ++s)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        ua[nb] = mfma_bf16_16x16x32(as_bf16x8(f.w[s]),
                                    as_bf16x8(ld16(Sb + (16 * nb + l16) * KP + 32 * s + 8 * g4)), ua[nb]);
    if (c > 0) pu(ahead.p, b ^ 1);
    load(c + 2, ahead);
#pragma unroll
    for (int s = 0; s < D / 32; ++s)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        ocur[nb] = mfma_bf16_16x16x32(as_bf16x8(f.q[s]),
                                      as_bf16x8(ld16(Sb + (16 * nb + l16) * KP + 32 * s + 8 * g4)), ocur[nb]);
    // U[tok][dv] = U~ - W S^T, stored transposed (Ut[dv][tok]): four consecutive tokens per write
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const uint32_t w0 = f.u[2 * nb], w1 = f.u[2 * nb + 1];
      const float u0 = bf2f((uint16_t)w0) - ua[nb][0], u1 = bf2f((uint16_t)(w0 >> 16)) - ua[nb][1];
      const float u2 = bf2f((uint16_t)w1) - ua[nb][2], u3 = bf2f((uint16_t)(w1 >> 16)) - ua[nb][3];
      *reinterpret_cast<u32x2_t *>(Ut[b] + (16 * nb + l16) * CP + 16 * wave + 4 * g4) =
          u32x2_t{pack_bf2(u0, u1), pack_bf2(u2, u3)};
    }
    if (c > 0) write_o(b ^ 1);
    lds_barrier();  // Ut[b] and Os[b ^ 1] complete; every read of Sb and of Os[b] is done
    // (b) S = e^{G_C} S + U^T K^, then its bf16 copy
    const float decay = expf(__builtin_bit_cast(
        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f.g), C - 1)));
#pragma unroll
    for (int i = 0; i < 16; ++i) st[i] *= decay;
#pragma unroll
    for (int s = 0; s < C / 16; ++s)
      st = mfma_bf16_32x32x16(as_bf16x8(ld16(Ut[b] + l32 * CP + 16 * s + 8 * gl)), as_bf16x8(f.k[s]), st);
    write_sb();
    lds_barrier();
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) oprev[nb] = ocur[nb];
  };

  Frags f0, f1, f2;
  load(0, f0);
  asm volatile("" ::: "memory");  // chunk 0's loads all issue before chunk 1's, as in the loop
  load(1, f1);
  write_sb();
  lds_barrier();
  // three chunks per trip, so every register set has a fixed name: chunk c in f[c % 3]
  int c = 0;
  for (; c + 3 <= n_chunks; c += 3) {
    step(c, f0, f2);
    step(c + 1, f1, f0);
    step(c + 2, f2, f1);
  }
  if (c < n_chunks) step(c, f0, f2);
  if (c + 1 < n_chunks) step(c + 1, f1, f0);
  // the last chunk's P U: the loads past the end left every register set holding the last chunk
  if (n_chunks > 1) store_o(n_chunks - 2);
  pu(f0.p, (n_chunks - 1) & 1);
  write_o((n_chunks - 1) & 1);
  lds_barrier();
  store_o(n_chunks - 1);
  if (s_final) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int vr = 8 * (i >> 2) + 4 * gl + (i & 3);
      s_final[((int64_t)h * D + 32 * sl + vr) * D + 32 * wave + l32] = st[i];
    }
  }
  wait_vm_lds<0>();  // the loads of the two chunks past the end land before the wave ends
}

}  // namespace
}  // namespace vdnh3

namespace vdnh3 {
namespace {
#ifndef VDNH3_GDN_SEGMENT_BYTES
#define VDNH3_GDN_SEGMENT_BYTES (2048ll << 20)
#endif
#ifndef VDNH3_GDN_PIPE_SEGMENTS
#define VDNH3_GDN_PIPE_SEGMENTS 8
#endif
constexpr int64_t kGdnPipeMinChunks = 32;  // a pipelined segment is at least this many chunks
// Workspace bytes of one (chunk, head): W, U~, Q^, K^ ([64][D] bf16 each), P ([64][64] bf16), G (64 fp32).
int64_t gdn_chunk_head_bytes(int head_dim) {
  return 4 * (int64_t)kGdnC * head_dim * 2 + (int64_t)kGdnC * kGdnC * 2 + (int64_t)kGdnC * 4;
}
// Chunks per segment. A sequence of fewer than 2 kGdnPipeMinChunks chunks runs as one segment;
// a longer one in about VDNH3_GDN_PIPE_SEGMENTS segments (at least kGdnPipeMinChunks chunks each)
// whose prep and scan overlap on two streams, through two workspace buffers of at most
// VDNH3_GDN_SEGMENT_BYTES / 2 each, so the workspace stays bounded however long the sequence.
int64_t gdn_segment_chunks(int64_t chunks, int heads, int head_dim) {
  int64_t cap = VDNH3_GDN_SEGMENT_BYTES / 2 / (heads * gdn_chunk_head_bytes(head_dim));
  cap = cap < 1 ? 1 : cap;
  if (chunks < 2 * kGdnPipeMinChunks && chunks <= cap) return chunks;
  int64_t seg = (chunks + VDNH3_GDN_PIPE_SEGMENTS - 1) / VDNH3_GDN_PIPE_SEGMENTS;
  seg = seg < kGdnPipeMinChunks ? kGdnPipeMinChunks : seg;
  return seg < cap ? seg : cap;
}
// Workspace buffers: two when the sequence runs in more than one segment.
int gdn_buffers(int64_t chunks, int64_t seg) { return seg < chunks ? 2 : 1; }

// The segment geometry of a call and the places of its workspace parts: buffer b holds
// [W | U~ | Q^ | K^ | P | G] of the segments i with i % 2 == b; the fp32 state carried between
// segments ([heads][D][D], 16-byte aligned) follows the buffers.
struct GdnLayout {
  int chunks = 0, seg = 0, segments = 0;
  struct Buf {
    uint16_t *W, *U, *Q, *K, *P;
    float *G;
  } buf[2] = {};
  float *carry = nullptr;
};
void gdn_geometry(int tokens, int heads, int *chunks, int *seg, int *segments) {
  *chunks = (tokens + kGdnC - 1) / kGdnC;
  *seg = (int)gdn_segment_chunks(*chunks, heads, 128);
  *segments = (*chunks + *seg - 1) / *seg;
}
GdnLayout gdn_layout(int tokens, int heads, void *workspace) {
  constexpr int D = 128;
  GdnLayout L;
  gdn_geometry(tokens, heads, &L.chunks, &L.seg, &L.segments);
  const int64_t n = (int64_t)L.seg * heads;
  const int64_t buf_bytes = n * gdn_chunk_head_bytes(D);
  for (int b = 0; b < gdn_buffers(L.chunks, L.seg); ++b) {
    uint16_t *base = reinterpret_cast<uint16_t *>(static_cast<char *>(workspace) + b * buf_bytes);
    L.buf[b].W = base;
    L.buf[b].U = L.buf[b].W + n * GdnWs<D>::W;
    L.buf[b].Q = L.buf[b].U + n * GdnWs<D>::U;
    L.buf[b].K = L.buf[b].Q + n * GdnWs<D>::Q;
    L.buf[b].P = L.buf[b].K + n * GdnWs<D>::K;
    L.buf[b].G = reinterpret_cast<float *>(L.buf[b].P + n * GdnWs<D>::P);
  }
  L.carry = reinterpret_cast<float *>(static_cast<char *>(workspace) + gdn_buffers(L.chunks, L.seg) * buf_bytes);
  return L;
}
// Segment i covers chunks i seg ..: its tokens form an independent sequence whose initial state is the
// state segment i - 1 ended with (the chunk form restarts exactly at a chunk boundary).
void gdn_span(const GdnLayout &L, int tokens, int i, int64_t *t0, int *nc, int *nt) {
  const int c0 = i * L.seg;
  *nc = L.seg < L.chunks - c0 ? L.seg : L.chunks - c0;
  *t0 = (int64_t)c0 * kGdnC;
  *nt = (int)(tokens - *t0 < (int64_t)*nc * kGdnC ? tokens - *t0 : (int64_t)*nc * kGdnC);
}

int gdn_check_common(int tokens, int heads, int head_dim, const void *workspace, size_t workspace_bytes);
}  // namespace
}  // namespace vdnh3

extern "C" size_t vdnh3_gdn_workspace_bytes(int tokens, int heads, int head_dim) {
  if (tokens <= 0 || heads <= 0 || head_dim <= 0) return 0;
  const int64_t chunks = (tokens + vdnh3::kGdnC - 1) / vdnh3::kGdnC;
  const int64_t seg = vdnh3::gdn_segment_chunks(chunks, heads, head_dim);
  // one or two segment buffers, then the fp32 state carried between segments ([heads][D][D])
  return (size_t)(vdnh3::gdn_buffers(chunks, seg) * seg * heads * vdnh3::gdn_chunk_head_bytes(head_dim) +
                  (int64_t)heads * head_dim * head_dim * 4);
}

extern "C" int vdnh3_gdn_segments(int tokens, int heads, int head_dim) {
  if (tokens <= 0 || heads <= 0 || head_dim != 128) return 0;
  int chunks, seg, segments;
  vdnh3::gdn_geometry(tokens, heads, &chunks, &seg, &segments);
  return segments;
}

namespace vdnh3 {
namespace {
int gdn_check_common(int tokens, int heads, int head_dim, const void *workspace, size_t workspace_bytes) {
  VDNH3_HOST_CHECK(head_dim == 128, VDNH3_ERR_INVALID, "gdn: head_dim must be 128, got %d", head_dim);
  VDNH3_HOST_CHECK(tokens > 0 && heads > 0, VDNH3_ERR_INVALID, "gdn: tokens and heads must be positive");
  VDNH3_HOST_CHECK(workspace != nullptr && reinterpret_cast<uintptr_t>(workspace) % 16 == 0, VDNH3_ERR_INVALID,
                   "gdn: workspace must be non-null and 16-byte aligned");
  VDNH3_HOST_CHECK(workspace_bytes >= vdnh3_gdn_workspace_bytes(tokens, heads, head_dim), VDNH3_ERR_INVALID,
                   "gdn: workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
                   vdnh3_gdn_workspace_bytes(tokens, heads, head_dim));
  return VDNH3_OK;
}
}  // namespace
}  // namespace vdnh3

extern "C" int vdnh3_gdn_prep(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *k, int64_t k_row,
                              int64_t k_head, const uint16_t *v, int64_t v_row, int64_t v_head, const float *beta,
                              int64_t beta_row, const float *log_decay, int64_t decay_row, int tokens, int heads,
                              int head_dim, int segment, void *workspace, size_t workspace_bytes, void *stream) {
  using namespace vdnh3;
  int rc = gdn_check_common(tokens, heads, head_dim, workspace, workspace_bytes);
  if (rc) return rc;
  VDNH3_HOST_CHECK(q && k && v && beta && log_decay, VDNH3_ERR_INVALID, "gdn: null operand");
  VDNH3_HOST_CHECK(q_row % 8 == 0 && q_head % 8 == 0 && k_row % 8 == 0 && k_head % 8 == 0 && v_row % 8 == 0 &&
                       v_head % 8 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(k) % 16 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0,
                   VDNH3_ERR_INVALID, "gdn: q/k/v must be 16-byte aligned with strides multiple of 8");
  constexpr int D = 128;
  const GdnLayout L = gdn_layout(tokens, heads, workspace);
  VDNH3_HOST_CHECK(segment >= 0 && segment < L.segments, VDNH3_ERR_INVALID, "gdn: segment %d of %d", segment,
                   L.segments);
  int64_t t0;
  int nc, nt;
  gdn_span(L, tokens, segment, &t0, &nc, &nt);
  const GdnLayout::Buf &b = L.buf[segment & 1];
  hipLaunchKernelGGL(gdn_prep_kernel<D>, dim3(heads, nc), dim3(256), 0, static_cast<hipStream_t>(stream),
                     q + t0 * q_row, q_row, q_head, k + t0 * k_row, k_row, k_head, v + t0 * v_row, v_row, v_head,
                     beta + t0 * beta_row, beta_row, log_decay + t0 * decay_row, decay_row, nt, heads, b.W, b.U,
                     b.Q, b.K, b.P, b.G);
  return check_launch("gdn_prep");
}

extern "C" int vdnh3_gdn_scan(const float *initial_state, float *final_state, uint16_t *out, int64_t o_row,
                              int64_t o_head, int tokens, int heads, int head_dim, int segment, void *workspace,
                              size_t workspace_bytes, void *stream) {
  using namespace vdnh3;
  int rc = gdn_check_common(tokens, heads, head_dim, workspace, workspace_bytes);
  if (rc) return rc;
  VDNH3_HOST_CHECK(out != nullptr && o_row % 8 == 0 && o_head % 8 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0,
                   VDNH3_ERR_INVALID, "gdn: out must be 16-byte aligned with strides multiple of 8");
  constexpr int D = 128;
  const GdnLayout L = gdn_layout(tokens, heads, workspace);
  VDNH3_HOST_CHECK(segment >= 0 && segment < L.segments, VDNH3_ERR_INVALID, "gdn: segment %d of %d", segment,
                   L.segments);
  int64_t t0;
  int nc, nt;
  gdn_span(L, tokens, segment, &t0, &nc, &nt);
  const GdnLayout::Buf &b = L.buf[segment & 1];
  const auto pieces = [](const uint16_t *x) { return reinterpret_cast<const u32x4_t *>(x); };
  // each scan workgroup reads its state slice before it writes the same slice, so the carry between
  // segments is updated in place
  hipLaunchKernelGGL(gdn_scan_kernel<D>, dim3(heads, D / 32), dim3(256), 0, static_cast<hipStream_t>(stream),
                     pieces(b.W), pieces(b.U), pieces(b.Q), pieces(b.K), pieces(b.P), b.G, nc, nt, heads,
                     segment == 0 ? initial_state : L.carry, segment == L.segments - 1 ? final_state : L.carry,
                     out + t0 * o_row, o_row, o_head);
  return check_launch("gdn_scan");
}

extern "C" int vdnh3_gdn_chunk_fwd(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *k,
                                   int64_t k_row, int64_t k_head, const uint16_t *v, int64_t v_row, int64_t v_head,
                                   const float *beta, int64_t beta_row, const float *log_decay, int64_t decay_row,
                                   const float *initial_state, float *final_state, uint16_t *out, int64_t o_row,
                                   int64_t o_head, int tokens, int heads, int head_dim, void *workspace,
                                   size_t workspace_bytes, void *stream) {
  int rc = vdnh3::gdn_check_common(tokens, heads, head_dim, workspace, workspace_bytes);
  if (rc) return rc;
  VDNH3_HOST_CHECK(out != nullptr, VDNH3_ERR_INVALID, "gdn: null operand");
  const int segments = vdnh3_gdn_segments(tokens, heads, head_dim);
  for (int i = 0; i < segments; ++i) {
    if ((rc = vdnh3_gdn_prep(q, q_row, q_head, k, k_row, k_head, v, v_row, v_head, beta, beta_row, log_decay,
                             decay_row, tokens, heads, head_dim, i, workspace, workspace_bytes, stream)))
      return rc;
    if ((rc = vdnh3_gdn_scan(initial_state, final_state, out, o_row, o_head, tokens, heads, head_dim, i, workspace,
                             workspace_bytes, stream)))
      return rc;
  }
  return VDNH3_OK;
}
