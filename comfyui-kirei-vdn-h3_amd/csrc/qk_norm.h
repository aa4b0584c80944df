// RMSNorm over the head dim with the optional split-half RoPE of the hybrid block's q_norm /
// k_norm (vdn_h3/hybrid.py:271-292), shared by the standalone q/k pass (block.hip) and the
// window attention's fused K pre-pass and Q load (window_attn.hip), so that every path gives the
// same bits:
//
//   y_d = x_d * r * w_d,   r = 1 / sqrt(ss / D + eps),
//   ss  = sum over the D/8 chunks of 8 channels: per chunk c an fmaf chain p_c over its 8 channels,
//         then a pairwise tree ((p0 + p1) + (p2 + p3)) + ... in chunk order;
//   RoPE: for pairs (i, i + h), h = rot / 2, with the 2x2 matrix F_i = [[f00, f01], [f10, f11]] of
//         the row: out_i = fmaf(f00, y_i, f01 * y_{i+h}), out_{i+h} = fmaf(f10, y_i, f11 * y_{i+h});
//         channels >= rot pass unchanged. One rounding to bf16 at the end.
#pragma once

#include "common.h"

namespace vdnh3 {

// The fmaf chain of one 8-channel chunk.
__device__ __forceinline__ float chunk_sumsq(const float *x) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss = fmaf(x[j], x[j], ss);
  return ss;
}

// The tree over chunk partials when chunk c's partial sits in lane c of an aligned group of NC
// lanes (NC = D / 8): butterfly exchanges at distance 1, 2, 4, ... give every lane
// ((p0 + p1) + (p2 + p3)) + ... (each step adds its own and its partner's value; the addition
// is commutative, so both partners hold the same bits).
template <int NC>
__device__ __forceinline__ float group_tree_sum(float p) {
#pragma unroll
  for (int o = 1; o < NC; o <<= 1) p += __shfl_xor(p, o);
  return p;
}

// The same tree over NC = 2 * M chunk partials when chunk 2s + g sits in element s of lane half g
// (g = lane / 32) of a wavefront: first the pairs (2s, 2s + 1) across the half-waves through
// v_permlane32_swap, then the local pairwise tree over s.
template <int M>
__device__ __forceinline__ float halves_tree_sum(const float (&p)[M]) {
  float q[M];
#pragma unroll
  for (int s = 0; s < M; ++s) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(p[s]), __float_as_uint(p[s]), false, false);
    q[s] = __uint_as_float(r[0]) + __uint_as_float(r[1]);  // low half's chunk 2s plus high half's 2s + 1
  }
#pragma unroll
  for (int w = 1; w < M; w <<= 1)
#pragma unroll
    for (int s = 0; s < M; s += 2 * w) q[s] = q[s] + q[s + w];
  return q[0];
}

__device__ __forceinline__ float rms_factor(float ss, int dim, float eps) { return 1.f / sqrtf(ss / (float)dim + eps); }

// The rotation of one channel: y is the channel's normalised value, o its partner's, m the pair's
// matrix (f00 f01 f10 f11); `first` when the channel is i < h (else i + h).
__device__ __forceinline__ float rope_rotate(float y, float o, f32x4_t m, bool first) {
  return first ? fmaf(m[0], y, m[1] * o) : fmaf(m[2], o, m[3] * y);
}

}  // namespace vdnh3
