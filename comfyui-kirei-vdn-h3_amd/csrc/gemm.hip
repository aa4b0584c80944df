// NT GEMM for gfx950 on bf16, int8 and fp8 (OCP e4m3fn) MFMA with a fused epilogue:
//
//   C[m][n] = epi( sum_k A[m][k] * B[n][k] )          A: [M, K] (lda), B: [N, K] (ldb), K contiguous
//   epi(acc) = act( round_opt( acc * alpha * a_scale[m] * b_scale[n] + bias[n] ) )   (+ C_old when accumulating)
//
// It stands in for every projection of the hybrid block: F.linear in bf16 (gates, beta, the
// VDN to_out_linear, vdn_h3/projection.py:259-261), the fp8 `_scaled_mm(x_q, W_q^T, s_x, s_w)`
// (vdn_h3/fp8.py:254-262) and the W8A8 int8 projection with per-token x per-channel scales
// (the ComfyUI-native qkv_proj / out_proj of vdn_h3/hybrid.py:263, :535).
//
// Tiling: a workgroup of 8 wavefronts (two per SIMD, so that one wavefront's MFMAs issue while
// the other waits on LDS or the barrier) computes a 256x256 tile of C; wavefront w owns rows
// 128 * (w / 4) .. +128 and columns 64 * (w % 4) .. +64 as 4 x 2 blocks of 32x32 MFMA accumulators
// (six 16-byte LDS fragment reads feed eight independent MFMAs per k-step). The 4-wavefront form
// (128 x 128 per wavefront, one per SIMD) is kept behind VDNH3_GEMM_WAVES=4; the 8-wavefront form
// measured 2-8% faster on the int8 and fp8 projection shapes. K advances in
// stages of 64 bytes per row (32 bf16, 64 int8 or 64 fp8 elements):
//   bf16: v_mfma_f32_32x32x16_bf16, 2 k-steps of 32 bytes per stage
//   int8: v_mfma_i32_32x32x32_i8,   2 k-steps of 32 bytes
//   fp8 : v_mfma_f32_32x32x64_f8f6f4 (no block scales), 1 k-step of 64 bytes
// Every lane reads its A and B k-slices at the same byte offsets, so the products pair the
// same k whatever order the instruction assigns to the lane's bytes.
// Stages are loaded straight into LDS (global_load_lds), in one of two pipelines (GemmPipe):
//  - bf16 and fp8: stages of 64 bytes per row in a five-slot ring (160 KB, all of the CU's LDS);
//    each stage's k-steps issue the loads of the stage four ahead, evenly spaced between their
//    MFMAs, so the loads have three to four stages of MFMA time to land;
//  - int8: stages of 128 bytes per row (whole 128-byte lines, half the barriers per MFMA) in two
//    slots (128 KB); stage s issues the loads of stage s + 1 in its first three k-steps (of four),
//    and the barrier sits before the last one. Against the ring at the projection shapes, bit-
//    identical: -2.8 to -4.4% (qkv) and -4.0 to -4.7% (out) on two machines. For fp8 (two k-steps per
//    stage, so the loads had one k-step to land) the same pipeline, and one with the loads spread
//    over both k-steps and the barrier after the second, measured from -1.6% to +3.5%: not kept.
// One barrier per stage frees a slot and publishes the next stage; fragments are double-buffered
// in registers one k-step ahead, across that barrier too. 16-byte chunk c of stage row r is
// stored at a slot that makes the 16-lane fragment reads conflict-free (gemm_slot).
// Tiles are ordered so that the 32 workgroups resident on one XCD cover a 4 x 8 block of
// tiles and share their A and B panels in that XCD's L2.
#include <type_traits>

#include "common.h"

namespace vdnh3 {
namespace {

constexpr int kGemmBM = 256, kGemmBN = 256;
constexpr int kGemmKB = 128;    // K bytes per row that the host requires K * element size to be a multiple of
#ifndef VDNH3_GEMM_WAVES
#define VDNH3_GEMM_WAVES 8
#endif
constexpr int kGemmWaves = VDNH3_GEMM_WAVES;  // wavefronts per workgroup: 4 (one per SIMD) or 8 (two)
static_assert(kGemmWaves == 4 || kGemmWaves == 8, "4 or 8 wavefronts per GEMM workgroup");
constexpr int kGemmThreads = 64 * kGemmWaves;
// a wavefront owns 128 rows x (32 kGemmNJ) columns of the tile: 2 x 2 wavefronts of 128 x 128
// or 2 x 4 wavefronts of 128 x 64
constexpr int kGemmNJ = 16 / kGemmWaves;
constexpr int kGemmGroupM = 4;  // tile rows per grouping band (4 measured 1-3% faster than 2, 8 or 16)

enum GemmKind { kBF16 = 0, kI8 = 1, kF8 = 2 };

// The stage pipeline of each operand kind (see the file comment): SK K bytes per row and stage,
// SLOTS LDS slots, LOADS 16-byte loads per thread and stage (A and B), KS k-steps per stage
// (32 bytes per lane group for bf16 / int8, 64 for fp8).
template <int KIND>
struct GemmPipe {
  static constexpr int SK = KIND == kI8 ? 128 : 64;
  static constexpr int SLOTS = SK == 64 ? 5 : 2;
  static constexpr int LOADS = 2 * kGemmBM * (SK / 16) / kGemmThreads;
  static constexpr int KS = SK / (KIND == kF8 ? 64 : 32);
};
enum OutType { kOutBF16 = 0, kOutF32 = 1, kOutI32 = 2 };

struct GemmEpi {
  const float *a_scale;  // [M] or null
  const float *b_scale;  // [N] or null (a single value when b_scale_n == 1)
  int b_scale_n;
  int a_scale_n;
  float alpha;
  const void *bias;  // [N] or null
  int bias_bf16;
  int act;            // 0 none, 1 sigmoid
  int act_cols;       // with the sigmoid: it applies to columns n < act_cols only (0: every column)
  int out_type;       // OutType
  int accumulate;     // C += epi(acc)
  int round_linear;   // bf16 output: round the linear result to bf16 before the activation
  int vec;            // N % 4 == 0, ldc % 4 == 0 and C aligned for 4-element stores
};

__device__ __forceinline__ float sigmoidf_(float x) { return 1.f / (1.f + __expf(-x)); }

// LDS slot of 16-byte chunk c of stage row r: 16 consecutive rows read at one chunk column hit 16
// different 16-byte bank groups (4 chunks per 64-byte row: row % 4 x 4 slots; 8 chunks per
// 128-byte row: row % 2 x 8 slots)
template <int SK>
__host__ __device__ constexpr int gemm_slot(int r, int c) {
  return SK == 64 ? c ^ ((r >> 2) & 3) : c ^ ((r >> 1) & 7);
}

// MFMA operand reads: one k-step = 32 bytes per row (bf16 / int8, one 16-byte chunk per lane
// group) or 64 bytes (fp8, two chunks per lane group)
template <int KIND>
struct Frag {
  using type = typename std::conditional<KIND == kF8, i32x8_t, u32x4_t>::type;
};

// Epilogue. Each wavefront stages its 128 x 128 block of C through LDS 32 rows at a time
// (row-major, kEpiStride words per row: rows r and r + 4, written by the two lane halves of
// one MFMA register, land 32 banks apart) and reads it back as row segments: lane
// (h = lane / 32, c = lane % 32) takes columns 4c .. 4c+3 of row 2 it + h, so each row of the
// block leaves as one contiguous run. The staged words are the raw accumulator bits (int32
// for int8 operands, fp32 otherwise). ACT (sigmoid) and ACCUM are not combined by any caller
// (the launcher keeps them apart).
constexpr int kEpiStride = 32 * kGemmNJ + 8;
constexpr int kEpiWaveWords = 32 * kEpiStride;
constexpr int kEpiLanesPerRow = 8 * kGemmNJ;         // four columns per lane
constexpr int kEpiRowsPerPass = 64 / kEpiLanesPerRow;  // rows one pass of the wavefront covers

// Per-lane epilogue operands, loaded at the start of the kernel so that their latency hides
// behind the main loop: the scales of rows mb + lane and mb + 64 + lane of the wavefront's
// block, and the column scale (times alpha) and bias of the lane's four columns nb + 4 (lane % 32) + k.
struct EpiOperands {
  float row_scale[2];
  float col_scale[4];
  float bias[4];
};

__device__ __forceinline__ EpiOperands load_epi_operands(const GemmEpi &epi, int M, int N, int mb, int nb, int lane) {
  EpiOperands o;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int m = min(mb + 64 * h + lane, M - 1);
    o.row_scale[h] = epi.a_scale ? epi.a_scale[epi.a_scale_n == 1 ? 0 : m] : 1.f;
  }
  const int n = nb + 4 * (lane % kEpiLanesPerRow);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int nk = min(n + k, N - 1);
    o.col_scale[k] = epi.b_scale ? epi.alpha * epi.b_scale[epi.b_scale_n == 1 ? 0 : nk] : epi.alpha;
    o.bias[k] = !epi.bias ? 0.f
                : epi.bias_bf16 ? bf2f(static_cast<const uint16_t *>(epi.bias)[nk])
                                : static_cast<const float *>(epi.bias)[nk];
  }
  return o;
}

// Output stores, and the loads of the old values when accumulating, are non-temporal (the `nt`
// hint): the output streams through each XCD's L2 at 128 KB per tile, which would otherwise
// evict the A and B panels that the XCD's other workgroups are still reading (6-8% of the int8 /
// fp8 projection time, 2% more for the accumulating to_out_linear; bit-identical output).
template <typename V, typename P>
__device__ __forceinline__ void stream_store(V v, P *p) {
  __builtin_nontemporal_store(v, reinterpret_cast<V *>(p));
}
template <typename V, typename P>
__device__ __forceinline__ V stream_load(const P *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const V *>(p));
}

template <int OUT, bool ACT, bool ACCUM, bool INT_ACC, typename Acc>
__device__ __forceinline__ void store_block(const Acc (&acc)[4][kGemmNJ], uint32_t *stage, const GemmEpi &epi,
                                            const EpiOperands &eo, void *C, int64_t ldc, int M, int N, int mb,
                                            int nb, int lane) {
  const int l32 = lane & 31, g = lane >> 5;
  const int c0 = 4 * (lane % kEpiLanesPerRow), pr = lane / kEpiLanesPerRow, n = nb + c0;
  const bool vec = epi.vec && n < N;  // the host sets vec only when N % 4 == 0 and C allows 4-wide stores
  using old_t = typename std::conditional<OUT == kOutF32, f32x4_t, u32x2_t>::type;
  const bool round_linear = epi.round_linear;
  const int act_cols = epi.act_cols > 0 ? epi.act_cols : N;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // stage rows 32 i .. +32 of the block
#pragma unroll
    for (int j = 0; j < kGemmNJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        // element copied out first: __builtin_bit_cast of a vector-element lvalue reads
        // element 0 whatever the index
        const auto e = acc[i][j][r];
        const uint32_t w = __builtin_bit_cast(uint32_t, e);
        stage[(8 * (r >> 2) + 4 * g + (r & 3)) * kEpiStride + 32 * j + l32] = w;
      }
    asm volatile("" ::: "memory");  // LDS operations of one wavefront complete in order
    // rows kEpiRowsPerPass it + pr of the round in chunks of four passes; when accumulating, a
    // chunk's old values are loaded together before any of its stores
#pragma unroll 1
    for (int c4 = 0; c4 < 32 / kEpiRowsPerPass / 4; ++c4) {
      old_t old[4];
      if constexpr (ACCUM) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int m = mb + 32 * i + kEpiRowsPerPass * (4 * c4 + q) + pr;
          old[q] = old_t{};
          if (vec && m < M) {
            const int64_t off = (int64_t)m * ldc + n;
            if constexpr (OUT == kOutF32) old[q] = stream_load<f32x4_t>(static_cast<float *>(C) + off);
            else old[q] = stream_load<u32x2_t>(static_cast<uint16_t *>(C) + off);
          }
        }
      }
      // the chunk's staged rows and row scales (row 32 i + row of the block: scale held by
      // lane (32 i + row) % 64, entry i / 2), read before any of its arithmetic
      u32x4_t wq[4];
      float asq[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = kEpiRowsPerPass * (4 * c4 + q) + pr;
        wq[q] = *reinterpret_cast<const u32x4_t *>(stage + row * kEpiStride + c0);
        asq[q] = __shfl(eo.row_scale[i >> 1], 32 * (i & 1) + row);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = mb + 32 * i + kEpiRowsPerPass * (4 * c4 + q) + pr;
        if (m >= M || n >= N) continue;
        const int64_t off = (int64_t)m * ldc + n;
        const u32x4_t w = wq[q];
        const uint32_t wk[4] = {w.x, w.y, w.z, w.w};
        if constexpr (OUT == kOutI32) {
          if (vec) {
            stream_store(w, static_cast<int32_t *>(C) + off);
          } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
              if (n + k < N) static_cast<uint32_t *>(C)[off + k] = wk[k];
          }
        } else {
          float v[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            float x = INT_ACC ? (float)__builtin_bit_cast(int32_t, wk[k]) : __builtin_bit_cast(float, wk[k]);
            x *= asq[q];  // 1 without row scales
            x = x * eo.col_scale[k] + eo.bias[k];
            // bf16 output: rounding the linear value first only matters before the sigmoid (a
            // second rounding of a bf16 value, or the accumulation's own rounding, is exact)
            if constexpr (OUT == kOutBF16 && ACT) x = round_linear ? round_bf(x) : x;
            if constexpr (ACT) x = n + k < act_cols ? sigmoidf_(x) : x;
            v[k] = x;
          }
          if constexpr (OUT == kOutF32) {
            float *cp = static_cast<float *>(C) + off;
            if (vec) {
              f32x4_t o = {v[0], v[1], v[2], v[3]};
              if constexpr (ACCUM) o += old[q];
              stream_store(o, cp);
            } else {
#pragma unroll
              for (int k = 0; k < 4; ++k)
                if (n + k < N) cp[k] = ACCUM ? cp[k] + v[k] : v[k];
            }
          } else {
            uint16_t *cp = static_cast<uint16_t *>(C) + off;
            if (vec) {
              uint32_t lo, hi;
              if constexpr (ACCUM) {
                const u32x2_t o = old[q];
                lo = pack_bf2(bf2f(o.x & 0xffff) + round_bf(v[0]), bf2f(o.x >> 16) + round_bf(v[1]));
                hi = pack_bf2(bf2f(o.y & 0xffff) + round_bf(v[2]), bf2f(o.y >> 16) + round_bf(v[3]));
              } else {
                lo = pack_bf2(v[0], v[1]);
                hi = pack_bf2(v[2], v[3]);
              }
              stream_store(u32x2_t{lo, hi}, cp);
            } else {
#pragma unroll
              for (int k = 0; k < 4; ++k)
                if (n + k < N) cp[k] = f2bf(ACCUM ? bf2f(cp[k]) + round_bf(v[k]) : v[k]);
            }
          }
        }
      }
    }
    asm volatile("" ::: "memory");
  }
}

template <int KIND>
__global__ __launch_bounds__(kGemmThreads, 1) void gemm_nt_kernel(const uint8_t *__restrict__ A, int64_t lda_b,
                                                                   const uint8_t *__restrict__ B, int64_t ldb_b,
                                                                   void *__restrict__ C, int64_t ldc, int M, int N,
                                                                   int nkt, GemmEpi epi, int tiles_m, int tiles_n,
                                                                   int per_xcd, int total) {
  using Pipe = GemmPipe<KIND>;
  constexpr int kGemmSK = Pipe::SK, kGemmStages = Pipe::SLOTS, kGemmLoads = Pipe::LOADS, KS = Pipe::KS;
  constexpr int STAGE_BYTES = kGemmBM * kGemmSK;  // one 256-row stage of A or B (16 or 32 KB)
  __shared__ __attribute__((aligned(16))) uint8_t smem[2][kGemmStages][STAGE_BYTES];
  static_assert(4 * kEpiWaveWords * 4 <= (int)sizeof(smem), "epilogue staging must fit the ring");
  auto &As = smem[0];
  auto &Bs = smem[1];

  // XCD-aware tile order: workgroups are dealt round-robin over the 8 XCDs, so logical tile L
  // of XCD x is bid = 8 (L - x per_xcd) + x. Logical tiles walk bands of kGemmGroupM tile rows,
  // column by column, so concurrently resident workgroups share A rows and B columns.
  const int bid = blockIdx.x;
  const int L = (bid & 7) * per_xcd + (bid >> 3);
  if (L >= total) return;
  const int band = L / (kGemmGroupM * tiles_n);
  const int first_m = band * kGemmGroupM;
  const int band_m = min(kGemmGroupM, tiles_m - first_m);
  const int in_band = L - band * kGemmGroupM * tiles_n;
  const int tm = first_m + in_band % band_m, tn = in_band / band_m;
  const int m0 = tm * kGemmBM, n0 = tn * kGemmBN;

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int kWavesN = kGemmWaves / 2;  // wavefront columns of the tile
  const int wm = (wave / kWavesN) * 128, wn = (wave % kWavesN) * (32 * kGemmNJ);
  const int mb = m0 + wm, nb = n0 + wn;
  const EpiOperands eo = load_epi_operands(epi, M, N, mb, nb, lane);

  // Stage loads. A stage is SK bytes of K for the tile's 256 A rows and 256 B rows; LDS position
  // P (16-byte units) of an operand's stage is row P / CPR, slot P % CPR (CPR = SK / 16 chunks per
  // row) and holds the chunk gemm_slot maps to that slot. Load instruction q (0 .. kGemmLoads / 2
  // - 1) of an operand covers positions kGemmThreads q + tid, i.e. rows (kGemmThreads / CPR) q +
  // tid / CPR.
  // Rows past M (N) read the last row; their results are not stored.
  // The source of a load is a wave-uniform base (the tile's first row, advanced by the stage)
  // plus a per-lane 32-bit byte offset that stays the same for every stage (the host checks
  // that 256 rows of A and B span less than 4 GB).
  constexpr int CPR = kGemmSK / 16, kHalf = kGemmLoads / 2, kRowsPerLoad = kGemmThreads / CPR;
  const int lrow = tid / CPR;
  const int lchunk = gemm_slot<kGemmSK>(lrow, tid % CPR);  // the swizzle only sees row bits below kRowsPerLoad
  uint32_t a_off[kHalf], b_off[kHalf];
#pragma unroll
  for (int q = 0; q < kHalf; ++q) {
    a_off[q] = (uint32_t)((min(m0 + kRowsPerLoad * q + lrow, M - 1) - m0) * lda_b + lchunk * 16);
    b_off[q] = (uint32_t)((min(n0 + kRowsPerLoad * q + lrow, N - 1) - n0) * ldb_b + lchunk * 16);
  }
  const uint8_t *a_tile = A + (int64_t)m0 * lda_b, *b_tile = B + (int64_t)n0 * ldb_b;
  // load q (0 .. kGemmLoads - 1) of stage st into ring slot `slot`: A for q < kHalf, else B
  const uint32_t lds_wave = lds_address(&smem[0][0][0]) + wave * 64 * 16;
  auto load_part = [&](int st, int slot, int q) __device__ {
    const int64_t off = (int64_t)st * kGemmSK;
    const int i = q % kHalf;
    const uint32_t dst =
        lds_wave + (uint32_t)(((q / kHalf) * kGemmStages + slot) * STAGE_BYTES + i * kGemmThreads * 16);
    global_to_lds16_sbase((q >= kHalf ? b_tile : a_tile) + off, q >= kHalf ? b_off[i] : a_off[i], dst);
  };

  // fragment byte offsets inside an operand's stage (rows 32 i + l32 share l32's swizzle):
  // bf16 / int8 k-step ks reads chunk 2 ks + g (foff[ks][0]); fp8 reads chunks 4 ks + 2 g and
  // 4 ks + 2 g + 1 (foff[ks][0], foff[ks][1])
  constexpr int NCH = KIND == kF8 ? 2 : 1;
  int foff[KS][NCH];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int chunk = KIND == kF8 ? 4 * ks + 2 * g + c : 2 * ks + g;
      foff[ks][c] = l32 * kGemmSK + gemm_slot<kGemmSK>(l32, chunk) * 16;
    }

  using acc_t = typename std::conditional<KIND == kI8, i32x16_t, f32x16_t>::type;
  acc_t acc[4][kGemmNJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < kGemmNJ; ++j) acc[i][j] = acc_t{};

  using frag_t = typename Frag<KIND>::type;
  frag_t fa[2][4], fb[2][kGemmNJ];
  // fragments of k-step ks of the stage in `slot` into buffer `buf`
  auto read_frags = [&](int slot, int ks, int buf) __device__ {
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t *at = smem[0][slot] + wm * kGemmSK;
    const uint8_t *bt = smem[1][slot] + wn * kGemmSK;
    auto rd = [&](const uint8_t *base, int i) __device__ {
      if constexpr (KIND == kF8) {
        const u32x4_t lo = ld16(base + i * 32 * kGemmSK + foff[ks][0]);
        const u32x4_t hi = ld16(base + i * 32 * kGemmSK + foff[ks][NCH - 1]);
        return frag_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      } else {
        return frag_t(ld16(base + i * 32 * kGemmSK + foff[ks][0]));
      }
    };
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[buf][i] = rd(at, i);
      if (i < kGemmNJ) fb[buf][i] = rd(bt, i);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // the 4 kGemmNJ MFMAs of one k-step; stage loads qa .. qb - 1 of stage ld_st sit between them,
  // evenly spaced (qa, qb are constants once the k-step loops are unrolled); `reads` (the next
  // k-step's fragment reads) follows the second MFMA, so that any LDS wait before the first ones
  // covers only older reads
  auto mfmas = [&](int buf, int ld_st, int ld_slot, int qa, int qb, auto reads) __device__ {
    constexpr int NM = 4 * kGemmNJ;
    const int nl = qb - qa;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < kGemmNJ; ++j) {
        const int mi = kGemmNJ * i + j;
        if (mi == 2) reads();
#pragma unroll
        for (int q = 0; q < kGemmLoads; ++q)
          if (q < nl && mi == (q * NM) / nl) load_part(ld_st, ld_slot, qa + q);
        // fixed issue order: each stage load sits between two MFMAs
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (KIND == kF8)
          // scale operands 0 select the unscaled v_mfma_f32_32x32x64_f8f6f4 (no scale VGPRs to read; the
          // same bits as unit E8M0 scales, 127): 0.6% faster on the projection shapes
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[buf][i], fb[buf][j], acc[i][j], 0, 0, 0, 0,
                                                                     0, 0);
        else if constexpr (KIND == kBF16)
          acc[i][j] = mfma_bf16_32x32x16(as_bf16x8(fa[buf][i]), as_bf16x8(fb[buf][j]), acc[i][j]);
        else
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4_t, fa[buf][i]),
                                                            __builtin_bit_cast(i32x4_t, fb[buf][j]), acc[i][j], 0, 0, 0);
      }
    __builtin_amdgcn_sched_barrier(0);
  };

  // Ring of kGemmStages = 5 slots; stage s lives in slot s % 5. Stage s's first k-step
  // fragments are read before it starts (buffer (KS s) % 2). Its k-steps issue the loads of
  // stage s + 4 into slot (s + 4) % 5, which every wave finished reading before the barrier of
  // stage s - 1. Before its last k-step, once this wave's reads of stage s are done and stage
  // s + 1 has landed, one barrier lets stage s + 1 be read (its first fragments are read
  // during the last k-step) and frees slot s % 5. At that barrier the loads issued after
  // stage s + 1's are those of stages s + 2, s + 3 and the first KS - 1 k-steps of stage s + 4.
  const int nst = nkt * (kGemmKB / kGemmSK);  // even for the ring
  if constexpr (kGemmStages == 5) {
  auto run_stage = [&](int s, int slot, auto parity, auto dma, auto next) __device__ {
    constexpr int P = decltype(parity)::value;
    const int ld_slot = slot == 0 ? kGemmStages - 1 : slot - 1;
    const int nslot = slot == kGemmStages - 1 ? 0 : slot + 1;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int buf = (P * KS + ks) & 1;
      const int q0 = ks * (kGemmLoads / KS), q1 = decltype(dma)::value ? q0 + kGemmLoads / KS : q0;
      if (ks + 1 < KS) {
        mfmas(buf, s + 4, ld_slot, q0, q1, [&]() __device__ { read_frags(slot, ks + 1, buf ^ 1); });
      } else if constexpr (decltype(next)::value) {
        if (decltype(dma)::value) wait_vm_lds<2 * kGemmLoads + kGemmLoads / KS * (KS - 1)>();
        else wait_vm_lds<0>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's reads of stage s are done
        bare_barrier();
        mfmas(buf, s + 4, ld_slot, q0, q1, [&]() __device__ { read_frags(nslot, 0, buf ^ 1); });
      } else {
        mfmas(buf, s + 4, ld_slot, q0, q1, []() __device__ {});
      }
    }
  };
  using T = std::true_type;
  using F = std::false_type;

  // prologue: stages 0..3 in flight, stage 0's first fragments read
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    if (st < nst) {
#pragma unroll
      for (int q = 0; q < kGemmLoads; ++q) load_part(st, st, q);
    }
  }
  if (nst >= 4) wait_vm_lds<3 * kGemmLoads>();
  else wait_vm_lds<0>();
  bare_barrier();
  read_frags(0, 0, 0);
  // stages in pairs (so that the fragment buffer parity is static); the last two pairs issue
  // no loads and the very last stage has no successor
  int s = 0, slot = 0;
  auto adv = [&]() __device__ { slot = slot == kGemmStages - 1 ? 0 : slot + 1; ++s; };
  for (; s + 4 < nst;) {
    run_stage(s, slot, std::integral_constant<int, 0>{}, T{}, T{});
    adv();
    run_stage(s, slot, std::integral_constant<int, 1>{}, T{}, T{});
    adv();
  }
  for (; s + 2 < nst;) {
    run_stage(s, slot, std::integral_constant<int, 0>{}, F{}, T{});
    adv();
    run_stage(s, slot, std::integral_constant<int, 1>{}, F{}, T{});
    adv();
  }
  run_stage(s, slot, std::integral_constant<int, 0>{}, F{}, T{});
  adv();
  run_stage(s, slot, std::integral_constant<int, 1>{}, F{}, F{});
  } else {
  // Two slots; stage s lives in slot s % 2 and issues the loads of stage s + 1 into the other slot,
  // where every wave finished reading stage s - 1 before the barrier of stage s - 1. The loads go
  // out in k-steps 0 .. KS - 2; before the last k-step (whose fragments were read during the one
  // before), once stage s + 1 has landed, one barrier publishes it and frees slot s % 2, and the
  // last k-step reads stage s + 1's first fragments.
  constexpr int kPer = (kGemmLoads + KS - 2) / (KS - 1);  // loads per k-step
  static_assert(KS % 2 == 0 && KS > 1, "the fragment buffer parity is the k-step's");
  auto run_stage = [&](int s, auto next) __device__ {
    const int slot = s & 1, nslot = slot ^ 1;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int buf = ks & 1;
      const int qa = decltype(next)::value ? min(ks * kPer, kGemmLoads) : 0;
      const int qb = decltype(next)::value ? min((ks + 1) * kPer, kGemmLoads) : 0;
      if (ks + 1 < KS) {
        mfmas(buf, s + 1, nslot, qa, qb, [&]() __device__ { read_frags(slot, ks + 1, buf ^ 1); });
      } else if constexpr (decltype(next)::value) {
        wait_vm_lds<0>();
        bare_barrier();
        mfmas(buf, s + 1, nslot, 0, 0, [&]() __device__ { read_frags(nslot, 0, buf ^ 1); });
      } else {
        mfmas(buf, s + 1, nslot, 0, 0, []() __device__ {});
      }
    }
  };
  using T = std::true_type;
  using F = std::false_type;

  // prologue: stage 0 landed, its first fragments read
#pragma unroll
  for (int q = 0; q < kGemmLoads; ++q) load_part(0, 0, q);
  wait_vm_lds<0>();
  bare_barrier();
  read_frags(0, 0, 0);
  for (int s = 0; s + 1 < nst; ++s) run_stage(s, T{});
  run_stage(nst - 1, F{});
  }

  // epilogue, specialised on the output type, activation and accumulation (one uniform
  // branch here instead of per-element tests); the ring's LDS is reused for staging
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  bare_barrier();  // every wave is done reading the last stage
  uint32_t *stage = reinterpret_cast<uint32_t *>(&smem[0][0][0]) + wave * kEpiWaveWords;
  constexpr bool kInt = KIND == kI8;
  if (epi.out_type == kOutI32) {
    store_block<kOutI32, false, false, kInt>(acc, stage, epi, eo, C, ldc, M, N, mb, nb, lane);
  } else if (epi.out_type == kOutF32) {
    if (epi.act) store_block<kOutF32, true, false, kInt>(acc, stage, epi, eo, C, ldc, M, N, mb, nb, lane);
    else if (epi.accumulate) store_block<kOutF32, false, true, kInt>(acc, stage, epi, eo, C, ldc, M, N, mb, nb, lane);
    else store_block<kOutF32, false, false, kInt>(acc, stage, epi, eo, C, ldc, M, N, mb, nb, lane);
  } else {
    if (epi.act) store_block<kOutBF16, true, false, kInt>(acc, stage, epi, eo, C, ldc, M, N, mb, nb, lane);
    else if (epi.accumulate) store_block<kOutBF16, false, true, kInt>(acc, stage, epi, eo, C, ldc, M, N, mb, nb, lane);
    else store_block<kOutBF16, false, false, kInt>(acc, stage, epi, eo, C, ldc, M, N, mb, nb, lane);
  }
}

template <int KIND>
int launch_gemm(const void *A, int64_t lda, const void *B, int64_t ldb, void *C, int64_t ldc, int M, int N, int K,
                const GemmEpi &epi, hipStream_t stream) {
  const int eb = KIND == kBF16 ? 2 : 1;
  const int64_t kb = (int64_t)K * eb;
  VDNH3_HOST_CHECK(M > 0 && N > 0 && K > 0, VDNH3_ERR_INVALID, "gemm: M, N, K must be positive (%d, %d, %d)", M, N,
                   K);
  VDNH3_HOST_CHECK(kb % kGemmKB == 0, VDNH3_ERR_INVALID,
                   "gemm: K * element size must be a multiple of %d bytes (K=%d)", kGemmKB, K);
  VDNH3_HOST_CHECK((lda * eb) % 16 == 0 && (ldb * eb) % 16 == 0 && lda >= K && ldb >= K && ldc >= N,
                   VDNH3_ERR_INVALID, "gemm: leading dimensions must cover K/N and be 16-byte multiples");
  VDNH3_HOST_CHECK(reinterpret_cast<uintptr_t>(A) % 16 == 0 && reinterpret_cast<uintptr_t>(B) % 16 == 0,
                   VDNH3_ERR_INVALID, "gemm: A and B must be 16-byte aligned");
  VDNH3_HOST_CHECK((int64_t)kGemmBM * lda * eb < (int64_t(1) << 32) && (int64_t)kGemmBN * ldb * eb < (int64_t(1) << 32),
                   VDNH3_ERR_INVALID, "gemm: a 256-row panel of A or B must span less than 4 GB");
  const int tiles_m = (M + kGemmBM - 1) / kGemmBM, tiles_n = (N + kGemmBN - 1) / kGemmBN;
  const int total = tiles_m * tiles_n, per_xcd = (total + 7) / 8;
  hipLaunchKernelGGL(gemm_nt_kernel<KIND>, dim3(per_xcd * 8), dim3(kGemmThreads), 0, stream,
                     static_cast<const uint8_t *>(A), lda * eb, static_cast<const uint8_t *>(B), ldb * eb, C, ldc, M,
                     N, int(kb / kGemmKB), epi, tiles_m, tiles_n, per_xcd, total);
  return check_launch("gemm_nt");
}

}  // namespace
}  // namespace vdnh3

extern "C" int vdnh3_gemm(int kind, const void *A, int64_t lda, const void *B, int64_t ldb, void *C, int64_t ldc,
                          int M, int N, int K, const float *a_scale, int a_scale_n, const float *b_scale,
                          int b_scale_n, float alpha, const void *bias, int bias_bf16, int act, int out_type,
                          int accumulate, int round_linear, void *stream) {
  using namespace vdnh3;
  VDNH3_HOST_CHECK(A && B && C, VDNH3_ERR_INVALID, "gemm: null operand");
  VDNH3_HOST_CHECK(out_type >= kOutBF16 && out_type <= kOutI32, VDNH3_ERR_INVALID, "gemm: bad out_type %d", out_type);
  VDNH3_HOST_CHECK(out_type != kOutI32 || kind == kI8, VDNH3_ERR_INVALID, "gemm: int32 output needs int8 operands");
  VDNH3_HOST_CHECK(act == 0 || (act > 0 && (act & 1) && (act >> 1) <= N), VDNH3_ERR_INVALID,
                   "gemm: bad activation %d", act);
  VDNH3_HOST_CHECK(!(act && accumulate), VDNH3_ERR_INVALID, "gemm: a sigmoid epilogue cannot accumulate");
  VDNH3_HOST_CHECK(!a_scale || a_scale_n == 1 || a_scale_n == M, VDNH3_ERR_INVALID,
                   "gemm: a_scale must have 1 or M entries");
  VDNH3_HOST_CHECK(!b_scale || b_scale_n == 1 || b_scale_n == N, VDNH3_ERR_INVALID,
                   "gemm: b_scale must have 1 or N entries");
  const int esize = out_type == kOutBF16 ? 2 : 4;
  const int vec = N % 4 == 0 && ldc % 4 == 0 && reinterpret_cast<uintptr_t>(C) % (4 * esize) == 0;
  GemmEpi epi{a_scale, b_scale, b_scale_n, a_scale_n, alpha, bias, bias_bf16, act & 1, act >> 1, out_type, accumulate,
              round_linear, vec};
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (kind) {
    case kBF16:
      return launch_gemm<kBF16>(A, lda, B, ldb, C, ldc, M, N, K, epi, s);
    case kI8:
      return launch_gemm<kI8>(A, lda, B, ldb, C, ldc, M, N, K, epi, s);
    case kF8:
      return launch_gemm<kF8>(A, lda, B, ldb, C, ldc, M, N, K, epi, s);
    default:
      return set_error(VDNH3_ERR_INVALID, "gemm: unknown operand kind %d", kind);
  }
}
