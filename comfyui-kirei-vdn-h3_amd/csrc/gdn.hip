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
// gdn_prep_kernel (grid chunks x heads, fully parallel): K K^T and Q K^T on bf16 MFMA; the
// unit-triangular systems by fp32 forward substitution, one right-hand-side column per thread
// (W's 128 columns and U~'s 128 columns: no barrier inside the solve); writes W, U~, Q^ = e^G Q,
// K^T^ = (e^{G_C - G} K)^T, P = Q K^T o D (bf16) and G (fp32) for each chunk.
// gdn_scan_kernel (grid heads x dv/32, sequential over chunks): one workgroup carries a 32-row
// slice of the state in MFMA accumulators (fp32); per chunk U = U~ - W S^T, O = Q^ S^T + P U and
// S = e^{G_C} S + U^T K^, with the next chunk's operands loaded into registers during the step.
#include "common.h"

namespace vdnh3 {
namespace {

constexpr int kGdnC = 64;  // chunk length

template <int D>
struct GdnWs {  // per (chunk, head) workspace element counts
  static constexpr int64_t W = (int64_t)kGdnC * D, U = W, Q = W, K = W, P = (int64_t)kGdnC * kGdnC, G = kGdnC;
};

template <int D>
__global__ __launch_bounds__(256) void gdn_prep_kernel(
    const uint16_t *__restrict__ q, int64_t q_row, int64_t q_head, const uint16_t *__restrict__ k, int64_t k_row,
    int64_t k_head, const uint16_t *__restrict__ v, int64_t v_row, int64_t v_head, const float *__restrict__ beta,
    int64_t b_row, const float *__restrict__ lg, int64_t g_row, int T, int heads, uint16_t *__restrict__ Wo,
    uint16_t *__restrict__ Uo, uint16_t *__restrict__ Qo, uint16_t *__restrict__ Ko, uint16_t *__restrict__ Po,
    float *__restrict__ Go) {
  constexpr int C = kGdnC, KP = D + 8, CH = D / 8, AP = C + 1;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[C * KP], Qs[C * KP], Vs[C * KP];
  __shared__ float As[C * AP];
  __shared__ float Gs[C], Bs[C];
  const int c = blockIdx.x, h = blockIdx.y, t0 = c * C, n = min(C, T - t0);
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
  if (wave == 0) {  // inclusive prefix sum of the log-decay over the chunk
    float x = lane < n ? lg[(int64_t)(t0 + lane) * g_row + h] : 0.f;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float y = __shfl_up(x, o);
      if (lane >= o) x += y;
    }
    Gs[lane] = x;
    Bs[lane] = lane < n ? beta[(int64_t)(t0 + lane) * b_row + h] : 0.f;
  }
  __syncthreads();

  // K K^T and Q K^T: wave w owns the 32 x 32 block (w / 2, w % 2)
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
    uint16_t *pc = Po + ch * GdnWs<D>::P;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int m = 32 * mb + 8 * (i >> 2) + 4 * gl + (i & 3);
      const float dec = nn <= m ? expf(Gs[m] - Gs[nn]) : 0.f;
      As[m * AP + nn] = nn < m ? Bs[m] * dec * akk[i] : 0.f;
      pc[m * C + nn] = f2bf(aqk[i] * dec);
    }
  }
  __syncthreads();

  // (I + A) X = R by forward substitution, column `col` per thread: W (col < D) with
  // R = diag(b e^G) K, U~ (col >= D) with R = diag(b) V
  if (tid < 2 * D) {
    const int col = tid < D ? tid : tid - D;
    const bool is_w = tid < D;
    const uint16_t *src = is_w ? Ks : Vs;
    uint16_t *dst = (is_w ? Wo : Uo) + ch * GdnWs<D>::W + col;
    float x[C];
#pragma unroll
    for (int i = 0; i < C; ++i) {
      float r = Bs[i] * bf2f(src[i * KP + col]);
      if (is_w) r *= expf(Gs[i]);
#pragma unroll
      for (int j = 0; j < i; ++j) r = fmaf(-As[i * AP + j], x[j], r);
      x[i] = r;
      dst[(int64_t)i * D] = f2bf(r);
    }
  }
  // Q^ = e^G Q (rows) and K^T^ = (e^{G_C - G} K)^T ([D][C]), and G
  {
    const float gc = Gs[C - 1];
    uint16_t *qc = Qo + ch * GdnWs<D>::Q;
    uint16_t *kc = Ko + ch * GdnWs<D>::K;
    for (int e = tid; e < C * D; e += 256) {
      const int r = e / D, d = e - r * D;  // Q^ row-major: lanes walk d
      qc[e] = f2bf(bf2f(Qs[r * KP + d]) * expf(Gs[r]));
      const int dd = e / C, rr = e - dd * C;  // K^T^: lanes walk tokens
      kc[e] = f2bf(bf2f(Ks[rr * KP + dd]) * expf(gc - Gs[rr]));
    }
    if (tid < C) Go[ch * GdnWs<D>::G + tid] = Gs[tid];
  }
}

// One workgroup = head h, state rows (dv) 32 s .. 32 s + 31; wave w holds the state block of dk
// columns 32 w .. 32 w + 31 as one 32x32 MFMA accumulator (fp32).
template <int D>
__global__ __launch_bounds__(256) void gdn_scan_kernel(
    const uint16_t *__restrict__ Wi, const uint16_t *__restrict__ Ui, const uint16_t *__restrict__ Qi,
    const uint16_t *__restrict__ Ki, const uint16_t *__restrict__ Pi, const float *__restrict__ Gi, int n_chunks,
    int T, int heads, const float *__restrict__ s_init, float *__restrict__ s_final, uint16_t *__restrict__ out,
    int64_t o_row, int64_t o_head) {
  static_assert(D == 128, "the scan keeps one 32-column state block per wave: head_dim 128");
  constexpr int C = kGdnC, KP = D + 8, CP = C + 8, UP = 32 + 8;
  __shared__ __attribute__((aligned(16))) uint16_t Wl[C * KP], Ql[C * KP], Kt[D * CP], Pl[C * CP], Ul[C * UP];
  __shared__ __attribute__((aligned(16))) uint16_t Sb[32 * KP], Ut[32 * CP];
  __shared__ float Gl[C];
  const int h = blockIdx.x, sl = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, gl = lane >> 5;

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

  // operands of chunk c, 16-byte pieces: W, Q^ (C x D), K^T^ (D x C), P (C x C), U~ slice (C x 32), G
  constexpr int NW = C * D / 8, NP = C * C / 8, NU = C * 32 / 8;
  constexpr int NTOT = 3 * NW + NP + NU;               // 3072 + 512 + 256 = 3840
  constexpr int PER = (NTOT + 255) / 256;             // 15 per thread
  u32x4_t reg[PER];
  float greg = 0.f;
  auto fetch = [&](int c) __device__ {
    const int64_t ch = (int64_t)c * heads + h;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int e = tid + 256 * u;
      u32x4_t val = {0, 0, 0, 0};
      if (e < NW) val = ld16(Wi + ch * GdnWs<D>::W + 8 * e);
      else if (e < 2 * NW) val = ld16(Qi + ch * GdnWs<D>::Q + 8 * (e - NW));
      else if (e < 3 * NW) val = ld16(Ki + ch * GdnWs<D>::K + 8 * (e - 2 * NW));
      else if (e < 3 * NW + NP) val = ld16(Pi + ch * GdnWs<D>::P + 8 * (e - 3 * NW));
      else if (e < NTOT) {
        const int x = e - 3 * NW - NP, r = x >> 2, cc = x & 3;
        val = ld16(Ui + ch * GdnWs<D>::U + (int64_t)r * D + 32 * sl + 8 * cc);
      }
      reg[u] = val;
    }
    if (tid < C) greg = Gi[ch * GdnWs<D>::G + tid];
  };
  auto stash = [&]() __device__ {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int e = tid + 256 * u;
      if (e < NW) st16(Wl + (e >> 4) * KP + 8 * (e & 15), reg[u]);
      else if (e < 2 * NW) { const int x = e - NW; st16(Ql + (x >> 4) * KP + 8 * (x & 15), reg[u]); }
      else if (e < 3 * NW) { const int x = e - 2 * NW; st16(Kt + (x >> 3) * CP + 8 * (x & 7), reg[u]); }
      else if (e < 3 * NW + NP) { const int x = e - 3 * NW; st16(Pl + (x >> 3) * CP + 8 * (x & 7), reg[u]); }
      else if (e < NTOT) { const int x = e - 3 * NW - NP; st16(Ul + (x >> 2) * UP + 8 * (x & 3), reg[u]); }
    }
    if (tid < C) Gl[tid] = greg;
  };

  write_sb();
  fetch(0);
  stash();
  __syncthreads();
  for (int c = 0; c < n_chunks; ++c) {
    if (c + 1 < n_chunks) fetch(c + 1);  // in flight during the step
    // (a) waves 0, 1: U = U~ - W S^T for tokens 32 w ..; waves 2, 3: O = Q^ S^T for tokens 32 (w - 2) ..
    const int tb = wave & 1;
    f32x16_t acc = {};
    {
      const uint16_t *arow = (wave < 2 ? Wl : Ql) + (32 * tb + l32) * KP + 8 * gl;
#pragma unroll
      for (int s = 0; s < D / 16; ++s)
        acc = mfma_bf16_32x32x16(as_bf16x8(ld16(arow + 16 * s)), as_bf16x8(ld16(Sb + l32 * KP + 16 * s + 8 * gl)),
                                 acc);
    }
    if (wave < 2) {
      // U[tok][dv] = U~ - acc; stored transposed (Ut[dv][tok]), four consecutive tokens per write
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int tok = 32 * tb + 8 * i4 + 4 * gl;
        float u[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) u[e] = bf2f(Ul[(tok + e) * UP + l32]) - acc[4 * i4 + e];
        *reinterpret_cast<u32x2_t *>(Ut + l32 * CP + tok) = u32x2_t{pack_bf2(u[0], u[1]), pack_bf2(u[2], u[3])};
      }
    }
    __syncthreads();
    // (b) waves 2, 3: O += P U and store; every wave: S = e^{G_C} S + U^T K^
    if (wave >= 2) {
#pragma unroll
      for (int s = 0; s < C / 16; ++s)
        acc = mfma_bf16_32x32x16(as_bf16x8(ld16(Pl + (32 * tb + l32) * CP + 16 * s + 8 * gl)),
                                 as_bf16x8(ld16(Ut + l32 * CP + 16 * s + 8 * gl)), acc);
      const int t0 = c * C;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int tok = t0 + 32 * tb + 8 * (i >> 2) + 4 * gl + (i & 3);
        if (tok < T) out[(int64_t)tok * o_row + (int64_t)h * o_head + 32 * sl + l32] = f2bf(acc[i]);
      }
    }
    {
      const float decay = expf(Gl[C - 1]);
#pragma unroll
      for (int i = 0; i < 16; ++i) st[i] *= decay;
#pragma unroll
      for (int s = 0; s < C / 16; ++s)
        st = mfma_bf16_32x32x16(as_bf16x8(ld16(Ut + l32 * CP + 16 * s + 8 * gl)),
                                as_bf16x8(ld16(Kt + (32 * wave + l32) * CP + 16 * s + 8 * gl)), st);
    }
    __syncthreads();  // every read of this chunk's operands and of Sb / Ut is done
    write_sb();
    if (c + 1 < n_chunks) stash();
    __syncthreads();
  }
  if (s_final) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int vr = 8 * (i >> 2) + 4 * gl + (i & 3);
      s_final[((int64_t)h * D + 32 * sl + vr) * D + 32 * wave + l32] = st[i];
    }
  }
}

}  // namespace
}  // namespace vdnh3

extern "C" size_t vdnh3_gdn_workspace_bytes(int tokens, int heads, int head_dim) {
  if (tokens <= 0 || heads <= 0 || head_dim <= 0) return 0;
  const int64_t chunks = (tokens + vdnh3::kGdnC - 1) / vdnh3::kGdnC;
  const int64_t per = 4 * (int64_t)vdnh3::kGdnC * head_dim * 2 + (int64_t)vdnh3::kGdnC * vdnh3::kGdnC * 2 +
                      (int64_t)vdnh3::kGdnC * 4;
  return (size_t)(chunks * heads * per);
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
  constexpr int D = 128;
  const int chunks = (tokens + kGdnC - 1) / kGdnC;
  const int64_t n = (int64_t)chunks * heads;
  uint16_t *W = static_cast<uint16_t *>(workspace);
  uint16_t *U = W + n * GdnWs<D>::W;
  uint16_t *Qh = U + n * GdnWs<D>::U;
  uint16_t *Kt = Qh + n * GdnWs<D>::Q;
  uint16_t *P = Kt + n * GdnWs<D>::K;
  float *G = reinterpret_cast<float *>(P + n * GdnWs<D>::P);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(gdn_prep_kernel<D>, dim3(chunks, heads), dim3(256), 0, s, q, q_row, q_head, k, k_row, k_head,
                     v, v_row, v_head, beta, beta_row, log_decay, decay_row, tokens, heads, W, U, Qh, Kt, P, G);
  int rc = check_launch("gdn_prep");
  if (rc) return rc;
  hipLaunchKernelGGL(gdn_scan_kernel<D>, dim3(heads, D / 32), dim3(256), 0, s, W, U, Qh, Kt, P, G, chunks, tokens,
                     heads, initial_state, final_state, out, o_row, o_head);
  return check_launch("gdn_scan");
}
