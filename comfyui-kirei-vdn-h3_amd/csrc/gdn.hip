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
// that reads it) and G (fp32) for each chunk, as 16-byte stores.
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
// that a wavefront's 16-byte fragment pieces lie in lane order (1 KB per load instruction):
//  - W, Q^ (A operands, 8 k-steps) and P (4 k-steps): piece p of the block is lane p % 64 of
//    k-step (p / 64) % steps of row block p / (64 steps): row 32 (p / (64 steps)) + p % 32,
//    columns 16 ((p / 64) % steps) + 8 ((p / 32) % 2) .. + 7;
//  - K^ = e^{G_C - G} K (B operand of state block w): piece ((w, s), lane) holds tokens
//    16 s + 8 (lane / 32) .. + 7 of column 32 w + lane % 32;
//  - U~ (state slice sl, row block tb, half j): piece ((sl, tb, j), lane) holds, at element
//    4 i + e, row 32 tb + 8 (2 j + i) + 4 (lane / 32) + e of column 32 sl + lane % 32 (the layout
//    of a 32x32 MFMA accumulator, elements 8 j .. 8 j + 7).
__device__ __forceinline__ int gdn_a_row(int p, int steps = 8) { return 32 * (p / (64 * steps)) + (p & 31); }
__device__ __forceinline__ int gdn_a_col(int p, int steps = 8) { return 16 * ((p >> 6) % steps) + 8 * ((p >> 5) & 1); }

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
      kv = ld16(k + row * k_row + (int64_t)h * k_head + 8 * cc);
      qv = ld16(q + row * q_row + (int64_t)h * q_head + 8 * cc);
      vv = ld16(v + row * v_row + (int64_t)h * v_head + 8 * cc);
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
      const int p = tid + 256 * u, r = gdn_a_row(p), k0 = gdn_a_col(p);
      const u32x4_t x = ld16(Qs + r * KP + k0);
      const float sc = Eg[r];
      st16(qc + 8 * p,
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
      st16(kc + 8 * ((((d >> 5) * 4 + (tc >> 1)) << 6) + 32 * (tc & 1) + (d & 31)),
           u32x4_t{pack_bf2(y[0], y[1]), pack_bf2(y[2], y[3]), pack_bf2(y[4], y[5]), pack_bf2(y[6], y[7])});
    }
#pragma unroll
    for (int u = 0; u < C * (C / 8) / 256; ++u) {
      const int p = tid + 256 * u, r = gdn_a_row(p, C / 16), j0 = gdn_a_col(p, C / 16);
      st16(pc + 8 * p, ld16(Ps + r * PP + j0));
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
    // U~ leaves from the accumulators: wave w's block is the scan's state slice w, and its
    // accumulator element 8 j + e of row block mb is exactly piece ((w, mb, j), lane) element e
    uint16_t *uc = Uo + ch * GdnWs<D>::U;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const f32x16_t &a = au[mb];
        st16(uc + 8 * ((((wave * 2 + mb) * 2 + j) << 6) + lane),
             u32x4_t{pack_bf2(a[8 * j], a[8 * j + 1]), pack_bf2(a[8 * j + 2], a[8 * j + 3]),
                     pack_bf2(a[8 * j + 4], a[8 * j + 5]), pack_bf2(a[8 * j + 6], a[8 * j + 7])});
      }
    __syncthreads();  // every read of Ks is done: W replaces it
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = 32 * mb + 8 * (i >> 2) + 4 * gl + (i & 3);
        Ks[r * KP + 32 * wave + l32] = f2bf(aw[mb][i]);
      }
  }
  __syncthreads();
  {
    uint16_t *wc = Wo + ch * GdnWs<D>::W;
#pragma unroll
    for (int u = 0; u < C * CH / 256; ++u) {
      const int p = tid + 256 * u;
      st16(wc + 8 * p, ld16(Ks + gdn_a_row(p) * KP + gdn_a_col(p)));
    }
  }
}

// One workgroup = head h, state rows (dv) 32 sl .. 32 sl + 31, four wavefronts: waves 0, 1 form
// tokens 32 w .. 32 w + 31 of U = U~ - W S^T, waves 2, 3 tokens 32 (w - 2) .. of O = Q^ S^T + P U,
// and wave w carries the state block of dk columns 32 w .. 32 w + 31 as one 32x32 MFMA
// accumulator (fp32), S = e^{G_C} S + U^T K^. s_init and s_final may be the same buffer: a
// workgroup reads its slice of s_init before anything else and writes the same slice of s_final
// last.
//
// Every wavefront reads only its own part of a chunk's operands (half of W or of Q^ and P, its
// U~ rows, its K^ block), stored in its fragment order, so each wavefront loads them straight
// into registers (1 KB per load instruction), two chunks ahead: a ring of three register sets,
// which keeps two chunks' loads in flight behind the step that computes. The state's bf16 copy
// (Sb) and U (Ut, transposed) are exchanged through LDS; the outputs of chunk c go to LDS (Os) in
// step c and to global memory at the start of step c + 1 (one 16-byte store per thread).
template <int D>
__global__ __launch_bounds__(256) void gdn_scan_kernel(
    const u32x4_t *__restrict__ Wi, const u32x4_t *__restrict__ Ui, const u32x4_t *__restrict__ Qi,
    const u32x4_t *__restrict__ Ki, const u32x4_t *__restrict__ Pi, const float *__restrict__ Gi, int n_chunks,
    int T, int heads, const float *s_init, float *s_final, uint16_t *__restrict__ out,
    int64_t o_row, int64_t o_head) {
  static_assert(D == 128, "the scan keeps one 32-column state block per wave: head_dim 128");
  constexpr int C = kGdnC, KP = D + 8, CP = C + 8, OP = 32 + 8;
  __shared__ __attribute__((aligned(16))) uint16_t Sb[32 * KP], Ut[32 * CP], Os[C * OP];
  const int h = blockIdx.x, sl = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, gl = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), tb = wave & 1;
  const bool u_wave = wave < 2;

  // one chunk's operands of this wavefront: a = W (u waves) or Q^ (o waves) for its 32 tokens,
  // p = U~ (u waves, 2 pieces) or P (o waves, 4), k = K^ of its state block, g = G of lane
  struct Frags {
    u32x4_t a[D / 16], p[C / 16], k[C / 16];
    float g;
  };
  // Every wave issues the same load sequence (no branch: the compiler then tracks each register
  // set's loads exactly); the u waves' p[2], p[3] repeat their two U~ pieces and go unused.
  const u32x4_t *a_src = (u_wave ? Wi : Qi) + (tb * (D / 16) << 6) + lane;
  const u32x4_t *p_src = u_wave ? Ui + (((sl * 2 + tb) * 2) << 6) + lane : Pi + (tb * (C / 16) << 6) + lane;
  const u32x4_t *k_src = Ki + (wave * (C / 16) << 6) + lane;
  const int64_t p_chunk = u_wave ? GdnWs<D>::U / 8 : GdnWs<D>::P / 8;  // 16-byte pieces per block
  const int p_step = u_wave ? 1 : 3;                                   // piece s at 64 (s & p_step)
  auto load = [&](int c, Frags &f) __device__ {
    c = c < n_chunks ? c : n_chunks - 1;  // past the end: the last chunk again, never used
    const int64_t ch = (int64_t)c * heads + h;
    const int64_t o16 = ch * (GdnWs<D>::W / 8);  // 16-byte pieces per W / U~ / Q^ / K^ block
#pragma unroll
    for (int s = 0; s < D / 16; ++s) f.a[s] = a_src[o16 + 64 * s];
#pragma unroll
    for (int s = 0; s < C / 16; ++s) f.p[s] = p_src[ch * p_chunk + 64 * (s & p_step)];
#pragma unroll
    for (int s = 0; s < C / 16; ++s) f.k[s] = k_src[o16 + 64 * s];
    f.g = Gi[ch * GdnWs<D>::G + lane];  // a vector load: its wait is a vmcnt like the others
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
  // outputs of chunk c (in Os) to global memory: thread = (token tid / 4, 8 dv columns)
  auto store_o = [&](int c) __device__ {
    const int tk = tid >> 2, pc = tid & 3, tok = c * C + tk;
    const u32x4_t val = ld16(Os + tk * OP + 8 * pc);
    if (tok < T) st16(out + (int64_t)tok * o_row + (int64_t)h * o_head + 32 * sl + 8 * pc, val);
  };

  auto step = [&](int c, const Frags &f, Frags &ahead) __device__ {
    if (c > 0) store_o(c - 1);
    load(c + 2, ahead);
    // (a) waves 0, 1: U = U~ - W S^T for tokens 32 w ..; waves 2, 3: O = Q^ S^T for tokens 32 (w - 2) ..
    f32x16_t acc = {};
#pragma unroll
    for (int s = 0; s < D / 16; ++s)
      acc = mfma_bf16_32x32x16(as_bf16x8(f.a[s]), as_bf16x8(ld16(Sb + l32 * KP + 16 * s + 8 * gl)), acc);
    if (u_wave) {
      // U[tok][dv] = U~ - acc; stored transposed (Ut[dv][tok]), four consecutive tokens per write
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int tok = 32 * tb + 8 * i4 + 4 * gl;
        const u32x4_t &up = f.p[i4 >> 1];
        const uint32_t w0 = up[2 * (i4 & 1)], w1 = up[2 * (i4 & 1) + 1];
        const float u0 = bf2f((uint16_t)w0) - acc[4 * i4], u1 = bf2f((uint16_t)(w0 >> 16)) - acc[4 * i4 + 1];
        const float u2 = bf2f((uint16_t)w1) - acc[4 * i4 + 2], u3 = bf2f((uint16_t)(w1 >> 16)) - acc[4 * i4 + 3];
        *reinterpret_cast<u32x2_t *>(Ut + l32 * CP + tok) = u32x2_t{pack_bf2(u0, u1), pack_bf2(u2, u3)};
      }
    }
    lds_barrier();  // Ut complete; every read of Sb and of the Os of chunk c - 1 is done
    // (b) waves 2, 3: O += P U into Os; every wave: S = e^{G_C} S + U^T K^, then its bf16 copy
    if (!u_wave) {
#pragma unroll
      for (int s = 0; s < C / 16; ++s)
        acc = mfma_bf16_32x32x16(as_bf16x8(f.p[s]), as_bf16x8(ld16(Ut + l32 * CP + 16 * s + 8 * gl)), acc);
#pragma unroll
      for (int i = 0; i < 16; ++i) Os[(32 * tb + 8 * (i >> 2) + 4 * gl + (i & 3)) * OP + l32] = f2bf(acc[i]);
    }
    {
      const float decay = expf(__builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f.g), C - 1)));
#pragma unroll
      for (int i = 0; i < 16; ++i) st[i] *= decay;
#pragma unroll
      for (int s = 0; s < C / 16; ++s)
        st = mfma_bf16_32x32x16(as_bf16x8(ld16(Ut + l32 * CP + 16 * s + 8 * gl)), as_bf16x8(f.k[s]), st);
    }
    write_sb();
    lds_barrier();
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
// Workspace bytes of one (chunk, head): W, U~, Q^, K^T^ ([64][D] bf16 each), P ([64][64] bf16), G (64 fp32).
int64_t gdn_chunk_head_bytes(int head_dim) {
  return 4 * (int64_t)kGdnC * head_dim * 2 + (int64_t)kGdnC * kGdnC * 2 + (int64_t)kGdnC * 4;
}
// The sequence runs in segments of this many chunks, so that the workspace stays at about
// VDNH3_GDN_SEGMENT_BYTES (2 GiB: one segment up to ~57k tokens at 40 heads) however long the sequence.
// Segments small enough to stay in the 256 MB last-level cache between prep and scan were measured
// slower (2.49-3.0 ms against 2.41 at 40,688 x 40 x 128): the scan's wait is not HBM latency.
int64_t gdn_segment_chunks(int64_t chunks, int heads, int head_dim) {
  const int64_t seg = VDNH3_GDN_SEGMENT_BYTES / (heads * gdn_chunk_head_bytes(head_dim));
  return seg < 1 ? 1 : (seg > chunks ? chunks : seg);
}
}  // namespace
}  // namespace vdnh3

extern "C" size_t vdnh3_gdn_workspace_bytes(int tokens, int heads, int head_dim) {
  if (tokens <= 0 || heads <= 0 || head_dim <= 0) return 0;
  const int64_t chunks = (tokens + vdnh3::kGdnC - 1) / vdnh3::kGdnC;
  const int64_t seg = vdnh3::gdn_segment_chunks(chunks, heads, head_dim);
  // one segment's workspace, then the fp32 state carried between segments ([heads][D][D])
  return (size_t)(seg * heads * vdnh3::gdn_chunk_head_bytes(head_dim) + (int64_t)heads * head_dim * head_dim * 4);
}

extern "C" int vdnh3_gdn_chunk_fwd(const uint16_t *q, int64_t q_row, int64_t q_head, const uint16_t *k,
                                   int64_t k_row, int64_t k_head, const uint16_t *v, int64_t v_row, int64_t v_head,
                                   const float *beta, int64_t beta_row, const float *log_decay, int64_t decay_row,
                                   const float *initial_state, float *final_state, uint16_t *out, int64_t o_row,
                                   int64_t o_head, int tokens, int heads, int head_dim, void *workspace,
                                   size_t workspace_bytes, void *stream) {
  using namespace vdnh3;
  VDNH3_HOST_CHECK(head_dim == 128, VDNH3_ERR_INVALID, "gdn: head_dim must be 128, got %d", head_dim);
  VDNH3_HOST_CHECK(tokens > 0 && heads > 0, VDNH3_ERR_INVALID, "gdn: tokens and heads must be positive");
  VDNH3_HOST_CHECK(q && k && v && beta && log_decay && out && workspace, VDNH3_ERR_INVALID, "gdn: null operand");
  VDNH3_HOST_CHECK(workspace_bytes >= vdnh3_gdn_workspace_bytes(tokens, heads, head_dim), VDNH3_ERR_INVALID,
                   "gdn: workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
                   vdnh3_gdn_workspace_bytes(tokens, heads, head_dim));
  VDNH3_HOST_CHECK(q_row % 8 == 0 && q_head % 8 == 0 && k_row % 8 == 0 && k_head % 8 == 0 && v_row % 8 == 0 &&
                       v_head % 8 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(k) % 16 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
                   VDNH3_ERR_INVALID, "gdn: q/k/v and workspace must be 16-byte aligned with strides multiple of 8");
  VDNH3_HOST_CHECK(o_row % 8 == 0 && o_head % 8 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0,
                   VDNH3_ERR_INVALID, "gdn: out must be 16-byte aligned with strides multiple of 8");
  constexpr int D = 128;
  const int chunks = (tokens + kGdnC - 1) / kGdnC;
  const int seg = (int)gdn_segment_chunks(chunks, heads, D);
  const int64_t n = (int64_t)seg * heads;
  uint16_t *W = static_cast<uint16_t *>(workspace);
  uint16_t *U = W + n * GdnWs<D>::W;
  uint16_t *Qh = U + n * GdnWs<D>::U;
  uint16_t *Kt = Qh + n * GdnWs<D>::Q;
  uint16_t *P = Kt + n * GdnWs<D>::K;
  float *G = reinterpret_cast<float *>(P + n * GdnWs<D>::P);
  float *carry = G + n * GdnWs<D>::G;  // [heads][D][D] fp32 state between segments (16-byte aligned)
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Segment by segment: the segment's tokens form an independent sequence whose initial state is the
  // state the previous segment ended with (the chunk form restarts exactly at a chunk boundary). Each
  // scan workgroup reads its state slice before it writes the same slice, so the carry is updated in place.
  for (int c0 = 0; c0 < chunks; c0 += seg) {
    const int nc = seg < chunks - c0 ? seg : chunks - c0;
    const int64_t t0 = (int64_t)c0 * kGdnC;
    const int nt = (int)(tokens - t0 < (int64_t)nc * kGdnC ? tokens - t0 : (int64_t)nc * kGdnC);
    const bool first = c0 == 0, last = c0 + nc >= chunks;
    hipLaunchKernelGGL(gdn_prep_kernel<D>, dim3(heads, nc), dim3(256), 0, s, q + t0 * q_row, q_row, q_head,
                       k + t0 * k_row, k_row, k_head, v + t0 * v_row, v_row, v_head, beta + t0 * beta_row, beta_row,
                       log_decay + t0 * decay_row, decay_row, nt, heads, W, U, Qh, Kt, P, G);
    int rc = check_launch("gdn_prep");
    if (rc) return rc;
    const auto pieces = [](const uint16_t *b) { return reinterpret_cast<const u32x4_t *>(b); };
    hipLaunchKernelGGL(gdn_scan_kernel<D>, dim3(heads, D / 32), dim3(256), 0, s, pieces(W), pieces(U), pieces(Qh),
                       pieces(Kt), pieces(P), G, nc, nt, heads,
                       first ? initial_state : carry, last ? final_state : carry, out + t0 * o_row, o_row, o_head);
    rc = check_launch("gdn_scan");
    if (rc) return rc;
  }
  return VDNH3_OK;
}
