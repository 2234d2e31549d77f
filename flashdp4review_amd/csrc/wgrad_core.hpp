// Shared pieces of the clipped per-sample weight-gradient kernels: operand
// loaders and MFMA tile cores for gfx950, and the single-pass cooperative kernel
// template (instantiated per dtype in wgrad_fused_*.hip, launched from
// wgrad_clip.hip).  See wgrad_clip.hip for the algorithm.
#pragma once

#include "fdp_common.hpp"
#include "gemm_dma.hpp"
#include "host_cache.hpp"

namespace fdp {
namespace wg {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int NT = 256;

constexpr int kPermMax = 1024;  // workgroups whose order the single-pass launch sets
constexpr int kPairMax = 256;   // split products per single-pass launch

struct Args {
  const void* a;
  const void* b;
  int64_t B, K, M, N;
  int64_t sab, lda, sbb, ldb;
  int tiles_m, tiles_n;
  int spg;     // samples per group (pass B)
  int groups;  // number of groups (pass B)
  float* partials;  // [B, tiles]
  const float* factors;  // [B]
  int fac_parts;         // streamed clipped-sum pass: > 0: it forms the factors itself from
                         // partials [B, fac_parts] (in place of `factors`)
  float* group_out;      // [groups, M, N] fp32 when groups > 1
  void* out;
  int64_t ldo;
  int out_dtype;
  float out_scale;
  NoiseSrc noise;          // injected or drawn z (row-major [M, N])
  float noise_scale;
  // single-pass (fused) kernel
  int64_t units;          // tiles * B work units, unit u = (tile u/B, sample u%B)
  int nwg;                // workgroups of the cooperative grid
  unsigned* bar;          // grid barrier arrivals
  unsigned* epoch;        // launches of the single-pass kernel on this workspace (its tag is epoch + 1)
  unsigned* poison;       // tag of a launch one of whose bounded waits expired
  unsigned* tile_turn;    // [tiles] hand-over tickets for tiles shared by workgroups
  float* tile_acc;        // [nwg, BM*BN] bf16 per-group tile sums (row-major)
  int* err;               // status word: set when a bounded wait gives up (sticky, read by the host)
  unsigned spin_limit;    // polls before a grid wait gives up
  float C, clamp;
  const float* clip_args_dev;
  float* norms_out;       // optional [B]
  float* factors_out;     // optional [B]
  // single-pass kernel: this launch covers samples [chunk_b0, chunk_b0+chunk_nb)
  int64_t chunk_b0, chunk_nb;
  int chunk_first, chunk_last;
  float* chunk_acc;       // [M, N] fp32 running sum carried between chunks
  int gq, gr;             // groups per tile (gr tiles have gq + 1)
  uint16_t perm[kPermMax];  // hardware workgroup -> work list index
  // Split products (single pass): the last product of each "owner" list entry
  // is contracted over its first split_k1 k-tiles by the owner and over the
  // rest by a "helper" entry of another CU; the r-th owner (in list order)
  // pairs with the r-th helper.  split_k1 == 0: no split products.
  uint32_t owner_mask[kPermMax / 32];
  uint32_t helper_mask[kPermMax / 32];
  unsigned* pair_flag;    // [kPairMax] helper -> owner hand-over flags
  int split_k1;
  // The bias of operand a (bias_op 1) or b (bias_op 2), formed by the grouped
  // single-pass and the streamed clipped-sum kernels (see bias_finish):
  //   bias[c] = bias_scale * sum_b c'_b sum_k op_b[k, c] + bias_noise_scale * zb[c],
  //   c'_b = clip(||op_b||_F) with the weight's C and clamp.
  int bias_op;            // 0: no bias
  int bias_P;             // tiles along the other axis: partials per (column, sample)
  int64_t bias_len;       // M (bias_op 1) or N (bias_op 2)
  float* bias_part;       // [B, bias_P, bias_len] column sums over a tile's counted k-tiles
  float* bias_sq;         // [B, tiles] sums of squares over a tile's counted k-tiles
  void* bias_out;
  int bias_dtype;
  float bias_scale;
  NoiseSrc bias_noise;
  float bias_noise_scale;
  float* bias_norms;      // optional [B]: ||op_b||_F
  float* bias_factors;    // optional [B]: c'_b
};

// ------------------------------------------------------------------ 16-bit
// LDS tile: [128 rows][64 k] of 16-bit values, 128 bytes per row, in 8 chunks of
// 16 bytes whose position is XOR-swizzled by the row index.
__device__ __forceinline__ int lds16_off(int row, int chunk) {
  return row * 128 + ((chunk ^ ((row ^ (row >> 3)) & 7)) << 4);
}

template <class DT>
struct Core16 {
  using dtype = DT;
  static constexpr int BK = 64;
  static constexpr int TILE_BYTES = 128 * 128;  // one operand tile
  static constexpr int SMEM = 4 * TILE_BYTES;   // 2 operands x 2 buffers
  using Frag = uint4;

  // Operand stored [K, R] with R contiguous (row stride ld).  Thread t loads
  // rows k0+4*(t>>4)+i (i<4), columns r0+8*(t&15)..+7.
  template <bool VEC>
  __device__ static inline void load_kr(const uint16_t* src, int64_t ld, int64_t K, int64_t R,
                                        int64_t k0, int64_t r0, uint4 (&reg)[4]) {
    const int t = threadIdx.x;
    const int64_t r = r0 + (t & 15) * 8;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = k0 + (t >> 4) * 4 + i;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (k < K) {
        const uint16_t* p = src + k * ld + r;
        if (VEC && r + 8 <= R) {
          v = *reinterpret_cast<const uint4*>(p);
        } else {
          uint16_t e[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) e[j] = (r + j < R) ? p[j] : uint16_t(0);
          v.x = e[0] | (uint32_t(e[1]) << 16);
          v.y = e[2] | (uint32_t(e[3]) << 16);
          v.z = e[4] | (uint32_t(e[5]) << 16);
          v.w = e[6] | (uint32_t(e[7]) << 16);
        }
      }
      reg[i] = v;
    }
  }
  // Transpose the 4(k) x 8(r) register block into 8 rows of 4 k-values.
  __device__ static inline void store_kr(char* lds, const uint4 (&reg)[4]) {
    const int t = threadIdx.x;
    const int rc = t & 15, kq = t >> 4;
    const uint32_t w0[4] = {reg[0].x, reg[0].y, reg[0].z, reg[0].w};
    const uint32_t w1[4] = {reg[1].x, reg[1].y, reg[1].z, reg[1].w};
    const uint32_t w2[4] = {reg[2].x, reg[2].y, reg[2].z, reg[2].w};
    const uint32_t w3[4] = {reg[3].x, reg[3].y, reg[3].z, reg[3].w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      const uint32_t lo = __builtin_amdgcn_perm(w1[j >> 1], w0[j >> 1], sel);
      const uint32_t hi = __builtin_amdgcn_perm(w3[j >> 1], w2[j >> 1], sel);
      const int row = rc * 8 + j;
      *reinterpret_cast<uint2*>(lds + lds16_off(row, kq >> 1) + ((kq & 1) << 3)) =
          make_uint2(lo, hi);
    }
  }
  // Operand stored [R, K] with K contiguous: 16-byte chunks go straight to LDS.
  template <bool VEC>
  __device__ static inline void load_rk(const uint16_t* src, int64_t ld, int64_t K, int64_t R,
                                        int64_t k0, int64_t r0, uint4 (&reg)[4]) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = t + NT * i;
      const int64_t r = r0 + (c >> 3);
      const int64_t k = k0 + (c & 7) * 8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (r < R) {
        const uint16_t* p = src + r * ld + k;
        if (VEC && k + 8 <= K) {
          v = *reinterpret_cast<const uint4*>(p);
        } else {
          uint16_t e[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) e[j] = (k + j < K) ? p[j] : uint16_t(0);
          v.x = e[0] | (uint32_t(e[1]) << 16);
          v.y = e[2] | (uint32_t(e[3]) << 16);
          v.z = e[4] | (uint32_t(e[5]) << 16);
          v.w = e[6] | (uint32_t(e[7]) << 16);
        }
      }
      reg[i] = v;
    }
  }
  __device__ static inline void store_rk(char* lds, const uint4 (&reg)[4]) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = t + NT * i;
      *reinterpret_cast<uint4*>(lds + lds16_off(c >> 3, c & 7)) = reg[i];
    }
  }

  __device__ static inline f32x16 mfma(uint4 a, uint4 b, f32x16 c) {
    if constexpr (DT::code == FDP_BF16) {
      return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                     __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    } else {
      return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                    __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
  }
  // One BK=64 k-tile of the wave's 64x64 sub-tile.
  __device__ static inline void mma(const char* As, const char* Bs, f32x16 (&acc)[2][2], int wm,
                                    int wn, int lane) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int chunk = ks * 2 + (lane >> 5);
      const int rr = lane & 31;
      const uint4 a0 = *reinterpret_cast<const uint4*>(As + lds16_off(wm + rr, chunk));
      const uint4 a1 = *reinterpret_cast<const uint4*>(As + lds16_off(wm + 32 + rr, chunk));
      const uint4 b0 = *reinterpret_cast<const uint4*>(Bs + lds16_off(wn + rr, chunk));
      const uint4 b1 = *reinterpret_cast<const uint4*>(Bs + lds16_off(wn + 32 + rr, chunk));
      acc[0][0] = mfma(a0, b0, acc[0][0]);
      acc[0][1] = mfma(a0, b1, acc[0][1]);
      acc[1][0] = mfma(a1, b0, acc[1][0]);
      acc[1][1] = mfma(a1, b1, acc[1][1]);
    }
  }

  // acc += tile (m0, n0) of G_b over the whole contraction axis.
  template <int LAYOUT, bool VEC>
  __device__ static void gemm(const Args& p, int64_t bidx, int64_t m0, int64_t n0,
                              f32x16 (&acc)[2][2], char* smem) {
    const uint16_t* A = static_cast<const uint16_t*>(p.a) + bidx * p.sab;
    const uint16_t* Bm = static_cast<const uint16_t*>(p.b) + bidx * p.sbb;
    // Buffer c holds the A tile at smem + 2c*TILE_BYTES and the B tile right after.
#define FDP_AS(c) (smem + (c) * (2 * TILE_BYTES))
#define FDP_BS(c) (smem + (c) * (2 * TILE_BYTES) + TILE_BYTES)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int nk = static_cast<int>((p.K + BK - 1) / BK);
    uint4 ra[4], rb[4];
    if (LAYOUT == FDP_LAYOUT_TN) load_kr<VEC>(A, p.lda, p.K, p.M, 0, m0, ra);
    else load_rk<VEC>(A, p.lda, p.K, p.M, 0, m0, ra);
    load_kr<VEC>(Bm, p.ldb, p.K, p.N, 0, n0, rb);
    if (LAYOUT == FDP_LAYOUT_TN) store_kr(FDP_AS(0), ra);
    else store_rk(FDP_AS(0), ra);
    store_kr(FDP_BS(0), rb);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      const bool more = kt + 1 < nk;
      if (more) {
        const int64_t k0 = int64_t(kt + 1) * BK;
        if (LAYOUT == FDP_LAYOUT_TN) load_kr<VEC>(A, p.lda, p.K, p.M, k0, m0, ra);
        else load_rk<VEC>(A, p.lda, p.K, p.M, k0, m0, ra);
        load_kr<VEC>(Bm, p.ldb, p.K, p.N, k0, n0, rb);
      }
      mma(FDP_AS(cur), FDP_BS(cur), acc, wm, wn, lane);
      if (more) {
        if (LAYOUT == FDP_LAYOUT_TN) store_kr(FDP_AS(cur ^ 1), ra);
        else store_rk(FDP_AS(cur ^ 1), ra);
        store_kr(FDP_BS(cur ^ 1), rb);
      }
      __syncthreads();
    }
  }
};

// ------------------------------------------------------------------- fp32
// LDS tile: [16 k][128 r] floats, row stride 132 floats; MFMA 32x32x2 reads one
// float per lane per operand, consecutive lanes on consecutive r.
struct Core32 {
  static constexpr int BK = 16;
  static constexpr int LD = 132;
  static constexpr int TILE_BYTES = BK * LD * 4;
  static constexpr int SMEM = 4 * TILE_BYTES;

  template <bool VEC>
  __device__ static inline void load_kr(const float* src, int64_t ld, int64_t K, int64_t R,
                                        int64_t k0, int64_t r0, float4 (&reg)[2]) {
    const int t = threadIdx.x;
    const int64_t k = k0 + (t >> 4);
    const int64_t r = r0 + (t & 15) * 8;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      const int64_t ri = r + 4 * i;
      if (k < K) {
        const float* p = src + k * ld + ri;
        if (VEC && ri + 4 <= R) {
          v = *reinterpret_cast<const float4*>(p);
        } else {
          v.x = (ri + 0 < R) ? p[0] : 0.f;
          v.y = (ri + 1 < R) ? p[1] : 0.f;
          v.z = (ri + 2 < R) ? p[2] : 0.f;
          v.w = (ri + 3 < R) ? p[3] : 0.f;
        }
      }
      reg[i] = v;
    }
  }
  __device__ static inline void store_kr(char* lds, const float4 (&reg)[2]) {
    const int t = threadIdx.x;
    float* base = reinterpret_cast<float*>(lds) + (t >> 4) * LD + (t & 15) * 8;
    *reinterpret_cast<float4*>(base) = reg[0];
    *reinterpret_cast<float4*>(base + 4) = reg[1];
  }
  // [R, K] with K contiguous: thread t loads row r0+(t>>1), k = k0+8*(t&1)..+7.
  template <bool VEC>
  __device__ static inline void load_rk(const float* src, int64_t ld, int64_t K, int64_t R,
                                        int64_t k0, int64_t r0, float4 (&reg)[2]) {
    const int t = threadIdx.x;
    const int64_t r = r0 + (t >> 1);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int64_t k = k0 + (t & 1) * 8 + 4 * i;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (r < R) {
        const float* p = src + r * ld + k;
        if (VEC && k + 4 <= K) {
          v = *reinterpret_cast<const float4*>(p);
        } else {
          v.x = (k + 0 < K) ? p[0] : 0.f;
          v.y = (k + 1 < K) ? p[1] : 0.f;
          v.z = (k + 2 < K) ? p[2] : 0.f;
          v.w = (k + 3 < K) ? p[3] : 0.f;
        }
      }
      reg[i] = v;
    }
  }
  __device__ static inline void store_rk(char* lds, const float4 (&reg)[2]) {
    const int t = threadIdx.x;
    float* base = reinterpret_cast<float*>(lds) + (t >> 1);
    const int kb = (t & 1) * 8;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      base[(kb + 4 * i + 0) * LD] = reg[i].x;
      base[(kb + 4 * i + 1) * LD] = reg[i].y;
      base[(kb + 4 * i + 2) * LD] = reg[i].z;
      base[(kb + 4 * i + 3) * LD] = reg[i].w;
    }
  }
  __device__ static inline void mma(const char* As, const char* Bs, f32x16 (&acc)[2][2], int wm,
                                    int wn, int lane) {
    const float* A = reinterpret_cast<const float*>(As);
    const float* Bf = reinterpret_cast<const float*>(Bs);
    const int rr = lane & 31;
#pragma unroll
    for (int ks = 0; ks < BK / 2; ++ks) {
      const int k = ks * 2 + (lane >> 5);
      const float a0 = A[k * LD + wm + rr], a1 = A[k * LD + wm + 32 + rr];
      const float b0 = Bf[k * LD + wn + rr], b1 = Bf[k * LD + wn + 32 + rr];
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
    }
  }
  template <int LAYOUT, bool VEC>
  __device__ static void gemm(const Args& p, int64_t bidx, int64_t m0, int64_t n0,
                              f32x16 (&acc)[2][2], char* smem) {
    const float* A = static_cast<const float*>(p.a) + bidx * p.sab;
    const float* Bm = static_cast<const float*>(p.b) + bidx * p.sbb;
    // Buffer c holds the A tile at smem + 2c*TILE_BYTES and the B tile right after.
#define FDP_AS(c) (smem + (c) * (2 * TILE_BYTES))
#define FDP_BS(c) (smem + (c) * (2 * TILE_BYTES) + TILE_BYTES)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int nk = static_cast<int>((p.K + BK - 1) / BK);
    float4 ra[2], rb[2];
    if (LAYOUT == FDP_LAYOUT_TN) load_kr<VEC>(A, p.lda, p.K, p.M, 0, m0, ra);
    else load_rk<VEC>(A, p.lda, p.K, p.M, 0, m0, ra);
    load_kr<VEC>(Bm, p.ldb, p.K, p.N, 0, n0, rb);
    if (LAYOUT == FDP_LAYOUT_TN) store_kr(FDP_AS(0), ra);
    else store_rk(FDP_AS(0), ra);
    store_kr(FDP_BS(0), rb);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      const bool more = kt + 1 < nk;
      if (more) {
        const int64_t k0 = int64_t(kt + 1) * BK;
        if (LAYOUT == FDP_LAYOUT_TN) load_kr<VEC>(A, p.lda, p.K, p.M, k0, m0, ra);
        else load_rk<VEC>(A, p.lda, p.K, p.M, k0, m0, ra);
        load_kr<VEC>(Bm, p.ldb, p.K, p.N, k0, n0, rb);
      }
      mma(FDP_AS(cur), FDP_BS(cur), acc, wm, wn, lane);
      if (more) {
        if (LAYOUT == FDP_LAYOUT_TN) store_kr(FDP_AS(cur ^ 1), ra);
        else store_rk(FDP_AS(cur ^ 1), ra);
        store_kr(FDP_BS(cur ^ 1), rb);
      }
      __syncthreads();
    }
  }
};

#undef FDP_AS
#undef FDP_BS

__device__ __forceinline__ void zero(f32x16 (&acc)[2][2]) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
}

// Output coordinates of accumulator element r of block (i, j) for this lane:
// 32x32 MFMA result layout, col = lane%32, row = 8*(r/4) + 4*(lane/32) + r%4.
__device__ __forceinline__ int acc_row(int wm, int i, int lane, int r) {
  return wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}
__device__ __forceinline__ int acc_col(int wn, int j, int lane) { return wn + 32 * j + (lane & 31); }

// Tile id -> output tile, in bands of kBandRows tile rows walked column by
// column: consecutive ids (which the XCD-aware workgroup numbering keeps on
// one XCD) form compact blocks that share A and B panels in that XCD's L2.
constexpr int kBandRows = 8;
__device__ __forceinline__ void tile_coords(const Args& p, int tile, int64_t& m0, int64_t& n0) {
  const int per_band = kBandRows * p.tiles_n;
  const int band = tile / per_band, in_band = tile % per_band;
  const int rows_left = p.tiles_m - band * kBandRows;
  const int band_rows = rows_left < kBandRows ? rows_left : kBandRows;
  m0 = int64_t(band * kBandRows + in_band % band_rows) * BM;
  n0 = int64_t(in_band / band_rows) * BN;
}

// ============================================================ bias of an operand
// The bias gradient of a DP layer is a clipped sum of the column sums of one
// operand of the weight gradient's product (grad_output: operand a of a
// Linear, G_b = g_b^T x_b; operand b of a Conv1D, G_b = x_b^T g_b):
//   bias[c] = bias_scale * sum_b c'_b sum_k op_b[k, c] + bias_noise_scale * zb[c],
//   c'_b = clip(||op_b||_F)           (flashdp/core/linear_clip.py:116-123).
// The product kernels take it from the operand fragments their MFMAs already
// hold, so grad_output is read once.  A 16-bit fragment pair gives its column
// sum and its square in two v_dot2 (with ones, and with itself).  Each element
// is counted once: in the tile grid, k-tile kt of a sample is counted by the
// tile whose index along the other axis is kt % P (P tiles there), and of the
// two waves that share a row (or column) of fragments, each sums half of them
// over every k-step of a counted k-tile.  The kernels pick the k-tile code
// with or without this work per k-tile: a branch inside the unrolled k-steps
// would keep the next step's LDS reads from being scheduled among this step's
// MFMAs, and VALU work on every k-tile competes with the MFMAs for issue.  A
// tile's column sums go to bias_part[b][other][c] (a row of the tile's columns
// is contiguous), its sum of squares to bias_sq[b][tile].

// acc + x.lo + x.hi and acc + x.lo^2 + x.hi^2 for two packed 16-bit values.
template <class DT>
__device__ __forceinline__ float dot2_ones(uint32_t x, float acc) {
  if constexpr (DT::code == FDP_BF16) {
    typedef __attribute__((ext_vector_type(2))) __bf16 v2;
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, x),
                                           __builtin_bit_cast(v2, 0x3f803f80u), acc, false);
  } else {
    typedef __attribute__((ext_vector_type(2))) _Float16 v2;
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, x), __builtin_bit_cast(v2, 0x3c003c00u),
                                  acc, false);
  }
}
template <class DT>
__device__ __forceinline__ float dot2_self(uint32_t x, float acc) {
  if constexpr (DT::code == FDP_BF16) {
    typedef __attribute__((ext_vector_type(2))) __bf16 v2;
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, x), __builtin_bit_cast(v2, x),
                                           acc, false);
  } else {
    typedef __attribute__((ext_vector_type(2))) _Float16 v2;
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, x), __builtin_bit_cast(v2, x), acc, false);
  }
}

// One fragment (8 consecutive k-values of the tile's column `col`) into a
// lane's column sum cs and sum of squares sq; the tile's columns at or past
// `lim` (past the operand's width: they may hold the next row's values) are
// left out of the squares.
template <class DT>
__device__ __forceinline__ void bias_frag(const uint4& f, float& cs, float& sq, int col, int lim) {
  const uint32_t w4[4] = {f.x, f.y, f.z, f.w};
  float c = cs, q = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    c = dot2_ones<DT>(w4[e], c);
    q = dot2_self<DT>(w4[e], q);
  }
  cs = c;
  sq += col < lim ? q : 0.f;
}
// A counted k-tile's bias work, after its MFMAs are issued: this wave reads
// its NF fragments (f0 .. f0 + NF - 1 of its row of A fragments, or column
// of B fragments, from tile row / column w0) of every k-step again from the
// LDS stage -- the stage stays valid until the next k-tile's barrier -- and
// adds them to cs / sq.  The MFMA code of the k-tile is left as it is.
template <class DT, class G, int BOP, int NF>
__device__ inline void bias_from_stage(const FDP_LDS char* st, int w0, int f0, float (&cs)[NF],
                                       float& sq, int col0, int lim) {
  constexpr int R = BOP == 1 ? G::BM : G::BN;
  constexpr int ROW = BOP == 1 ? G::ROW_A : G::ROW_B;
  constexpr uint32_t base = BOP == 1 ? 0u : static_cast<uint32_t>(G::TILE_A);
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < NF; ++i) {
    const uint32_t o0 = dma::frag_off<R>(w0, f0 + i, 0) + base;
    const uint32_t o1 = dma::frag_off<R>(w0, f0 + i, 1) + base;
    uint4 fr[G::KS];
#pragma unroll
    for (int ks = 0; ks < G::KS; ++ks)
      fr[ks] = dma::read_frag(st, o0 + ks * 16 * ROW, o1 + ks * 16 * ROW);
#pragma unroll
    for (int ks = 0; ks < G::KS; ++ks) bias_frag<DT>(fr[ks], cs[i], sq, col0 + 32 * i + (lane & 31), lim);
  }
}
// Columns of the bias operand left in a tile that starts at column c0
// (clamped to 2^30: a tile is narrower).
__device__ __forceinline__ int bias_limit(int64_t len, int64_t c0) {
  const int64_t l = len - c0;
  return l < (int64_t(1) << 30) ? static_cast<int>(l) : (1 << 30);
}

// End of one sample's product in a 4-wave workgroup: a wave's column sums
// (lanes l and l + 32 hold the two k halves of one column) go to bcol at its
// columns cl0 + 32 f + lane (f < NF), its sum of squares to bred[wave]; both
// are cleared.  The caller then synchronises and calls bias_park or
// bias_store.
template <int NF>
__device__ __forceinline__ void bias_fold(float (&cs)[NF], float& sq, float* bcol, float* bred,
                                          int cl0) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const float v = cs[f] + __shfl_xor(cs[f], 32, kWave);
    if (lane < 32) bcol[cl0 + 32 * f + lane] = v;
    cs[f] = 0.f;
  }
  const float q = wave_sum_dpp(sq);
  if (lane == 0) bred[wave] = q;
  sq = 0.f;
}
// After the synchronisation that follows bias_fold: one product's partials
// into vals[0, W) and *sq (LDS, where they wait until the k-loop is over).
template <int W>
__device__ __forceinline__ void bias_park(const float* bcol, const float* bred, float* vals,
                                          float* sq) {
  for (int t = threadIdx.x; t < W; t += NT) vals[t] = bcol[t];
  if (threadIdx.x == 0) *sq = (bred[0] + bred[1]) + (bred[2] + bred[3]);
}
// The partials of sample b in tile `tile` (local columns [0, W) from column
// c0): one row of bias_part [B][P][len] (coalesced stores) and one bias_sq
// entry.
template <int W>
__device__ __forceinline__ void bias_store(const Args& p, const float* vals, float sq, int64_t b,
                                           int tile, int tiles, int64_t c0, int other) {
  float* row = p.bias_part + (b * p.bias_P + other) * p.bias_len + c0;
  for (int t = threadIdx.x; t < W; t += NT) {
    if (c0 + t < p.bias_len) st_coherent(row + t, vals[t]);
  }
  if (threadIdx.x == 0) st_coherent(p.bias_sq + b * tiles + tile, sq);
}

// Outputs [wg * kBiasCols, ...) (and every nwg * kBiasCols after) of the bias
// from the partials of all B samples.  A workgroup first forms the clip
// factors of up to kBiasFacBlock samples into LDS (L = NT / samples threads
// per sample, each summing a strided part of the sample's tiles, then a
// butterfly over the L lanes), then kBiasLanes threads per output each add
// c'_b * partial over a contiguous range of the (sample, partial) pairs, and
// the ranges are added in order: a fixed summation order for a given shape,
// so the result is deterministic.  Every load of a round is issued before
// any is used (one round trip for the factors, one for the partials).
// Workgroup 0 writes bias_norms / bias_factors.  Every thread of the
// workgroup calls it.
constexpr int kBiasCols = 16;
constexpr int kBiasLanes = NT / kBiasCols;  // threads per output
constexpr int kBiasFacBlock = NT;
struct BiasSmem {
  float fac[kBiasFacBlock];
  float red[NT];
};
__device__ inline void bias_factors(const Args& p, int tiles, int64_t fb, int nb, bool writer,
                                    bool poisoned, float C, float clamp, float* fac) {
  int L = kWave;
  while (L > 1 && L * nb > NT) L >>= 1;  // power of two: a sample's lanes lie in one wavefront
  const int s = threadIdx.x / L, r = threadIdx.x % L;
  float v = 0.f;
  if (s < nb) {
    const float* sq = p.bias_sq + (fb + s) * tiles;
    for (int t0 = r; t0 < tiles; t0 += 8 * L) {
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = t0 + e * L < tiles ? ld_coherent(sq + t0 + e * L) : 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) v += x[e];
    }
  }
  for (int off = L >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  if (s < nb && r == 0) {
    const float n = poisoned ? __builtin_nanf("") : sqrtf(v);
    const float cf = poisoned ? n : clip_factor(n, C, clamp);
    fac[s] = cf;
    if (writer) {
      if (p.bias_norms) p.bias_norms[fb + s] = n;
      if (p.bias_factors) p.bias_factors[fb + s] = cf;
    }
  }
}
__device__ inline void bias_finish(const Args& p, int tiles, int wg, int nwg, bool poisoned,
                                   BiasSmem& sm) {
  const int q = threadIdx.x / kBiasCols, cl = threadIdx.x % kBiasCols;
  float C = p.C, clamp = p.clamp;
  if (p.clip_args_dev != nullptr) {
    C = p.clip_args_dev[0];
    clamp = p.clip_args_dev[1];
  }
  const int64_t B = p.B, len = p.bias_len;
  const int P = p.bias_P;
  for (int64_t c0 = int64_t(wg) * kBiasCols; c0 < len; c0 += int64_t(nwg) * kBiasCols) {
    const int64_t c = c0 + cl;
    float acc = 0.f;
    for (int64_t fb = 0; fb < B; fb += kBiasFacBlock) {
      const int nb = B - fb < kBiasFacBlock ? static_cast<int>(B - fb) : kBiasFacBlock;
      bias_factors(p, tiles, fb, nb, wg == 0 && c0 == 0, poisoned, C, clamp, sm.fac);
      __syncthreads();
      const int npair = nb * P;
      const int j0 = (q * npair) / kBiasLanes, j1 = ((q + 1) * npair) / kBiasLanes;
      if (c < len) {
        const float* src = p.bias_part + fb * P * len + c;  // pair j = (sample, partial) at j * len
        for (int j = j0; j < j1; j += 8) {
          float x[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = j + e < j1 ? ld_coherent(src + (j + e) * len) : 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (j + e < j1) acc += sm.fac[(j + e) / P] * x[e];
        }
      }
      __syncthreads();  // the factors are read before the next block replaces them
    }
    sm.red[threadIdx.x] = acc;
    __syncthreads();
    if (q == 0 && c < len) {
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < kBiasLanes; ++k) v += sm.red[k * kBiasCols + cl];
      v *= p.bias_scale;
      if (p.bias_noise.on()) v += p.bias_noise_scale * p.bias_noise.at(c);
      if (poisoned) v = __builtin_nanf("");
      store_from_f32(p.bias_out, c, p.bias_dtype, v);
    }
    __syncthreads();
  }
}

// The bias from the partials of a completed launch (the streamed schedule).
template <int kUnused = 0>
__global__ __launch_bounds__(NT) void bias_finish_kernel(Args p, int tiles) {
  __shared__ BiasSmem sm;
  bias_finish(p, tiles, blockIdx.x, gridDim.x, false, sm);
}

// ============================================================ single pass
// Cross-workgroup exchange in the single-pass kernel.  Values that another
// workgroup reads (per-tile partial norms, per-group tile sums) are written and
// read as relaxed agent-scope atomics: on gfx950 these are coherent (sc1)
// accesses that bypass the per-XCD L2s, so no L2 write-back / invalidate fence
// is needed; ordering against the counters comes from an explicit
// s_waitcnt vmcnt(0) before each counter update.  Every wait is bounded
// (kSpinLimit polls); on expiry err is set and the kernel runs to completion,
// so no wave is ever left spinning.
constexpr unsigned kSpinLimit = 1u << 22;
// Poll interval of every inter-workgroup wait: s_sleep 16 (about 1000 clocks).
// All waiting workgroups poll one word; polling it faster congests the L2
// channel that holds it and slows the workgroups still computing.
constexpr int kPollSleep = 16;
constexpr int kXcds = 8;


// All workgroups of the (co-resident) grid arrive before any leaves.
// grid_wait returns (in every thread) whether this workgroup's results must be poisoned: its own
// wait expired, or an earlier wait of this launch did (that one stored the
// launch's tag in *poison before this workgroup could arrive).
//
// The counter resets itself: the last arriver (arrival index n-1) stores 0 and
// leaves at once.  A waiter with arrival index i sees the counter in
// [i+1, n-1] until everyone has arrived, then n or (after the reset) 0, which
// is <= i: either ends its wait.  So the counter is zero again when the
// barrier is over, with no second counter to reset.  Every workgroup arrives
// exactly once, even after an expired wait, so this holds in every launch.
//
// Launch tags: every workgroup reads *epoch when it starts and uses tag =
// epoch + 1 for the hand-over flags and the poison word of this launch; the
// last arriver advances *epoch.  Every workgroup has started (and read the
// epoch) before the last one arrives, so a launch's workgroups agree on the
// tag, and a flag or poison word left by an earlier launch (for instance one
// whose wait expired) never carries the current tag: an expiry affects only
// the launch it happened in.
//
// quiet_until (a wall_clock64() value, 0 = none): before the first poll the
// waiting wave sleeps without touching memory until then.  Coherent polling
// loads stall the vector memory pipeline of their CU, so a workgroup that
// arrives early would otherwise slow the other workgroup still computing on
// its CU; callers pass an estimate of when the slowest workgroup arrives.
//
// Split in two: grid_arrive() (every thread; thread 0 gets the arrival index)
// and grid_wait(); a workgroup may do work of its own in between.  With
// epoch == nullptr the same pair waits for the n workgroups that share one
// counter (a part of the grid, all of which arrive once per launch); the
// launch epoch is then left alone.
__device__ inline unsigned grid_arrive(unsigned* bar) {
  wait_stores();
  __syncthreads();
  unsigned i = 0;
  if (threadIdx.x == 0)
    i = __hip_atomic_fetch_add(bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return i;
}
// Marks this launch (tag) as poisoned and sets the host's status word.
__device__ __forceinline__ void expire(int* err, unsigned* poison, unsigned tag) {
  atomicOr(err, 1);
  __hip_atomic_store(poison, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline bool grid_wait(unsigned* bar, unsigned n, unsigned i, int* err, unsigned* epoch,
                                 unsigned* poison, unsigned tag, unsigned limit, int* flag,
                                 uint64_t quiet_until = 0, int poll_sleep = kPollSleep) {
  if (threadIdx.x == 0) {
    int bad = 0;
    if (i + 1 == n) {
      __hip_atomic_store(bar, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (epoch != nullptr)
        __hip_atomic_fetch_add(epoch, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      while (wall_clock64() < quiet_until) __builtin_amdgcn_s_sleep(32);
      // at most `limit` polls (0: none -- the wait expires at once, which
      // tests use to force the expiry path deterministically)
      for (unsigned spins = 0;; ++spins) {
        if (spins >= limit) {
          expire(err, poison, tag);
          bad = 1;
          break;
        }
        const unsigned v = __hip_atomic_load(bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (v >= n || v <= i) break;
        if (poll_sleep >= 16) __builtin_amdgcn_s_sleep(16);
        else __builtin_amdgcn_s_sleep(2);
      }
    }
    if (!bad) bad = __hip_atomic_load(poison, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == tag;
    *flag = bad;
  }
  __syncthreads();
  return *flag != 0;
}

// Workgroups are dealt round-robin to the 8 XCDs; give each XCD a contiguous
// block of logical ids so that neighbouring work shares that XCD's L2.
__device__ __forceinline__ int logical_wg(int hw, int nwg) {
  if (nwg % kXcds != 0) return hw;
  return (hw % kXcds) * (nwg / kXcds) + hw / kXcds;
}

template <bool PACK>
struct Held;
template <>
struct Held<true> {  // 64 fp32 accumulators -> 32 bf16 pairs (RNE)
  uint32_t v[2][2][8];
  __device__ __forceinline__ void put(const f32x16 (&acc)[2][2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 8; ++q)
          v[i][j][q] = BF16::pack2(acc[i][j][2 * q], acc[i][j][2 * q + 1]);
  }
  __device__ __forceinline__ void add_to(f32x16 (&tot)[2][2], float c) const {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const uint32_t w = v[i][j][q];
          tot[i][j][2 * q] += c * __uint_as_float(w << 16);
          tot[i][j][2 * q + 1] += c * __uint_as_float(w & 0xffff0000u);
        }
  }
};
template <>
struct Held<false> {
  f32x16 v[2][2];
  __device__ __forceinline__ void put(const f32x16 (&acc)[2][2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) v[i][j] = acc[i][j];
  }
  __device__ __forceinline__ void add_to(f32x16 (&tot)[2][2], float c) const {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) tot[i][j][r] += c * v[i][j][r];
  }
};


// ------------------------------------------------------ single-pass work map
// A launch covers samples [chunk_b0, chunk_b0 + chunk_nb) with W workgroups.
// The workgroups form a tile-major list: tiles [0, gr) have gq + 1 groups,
// tiles [gr, tiles) have gq groups, and group g of a tile with ng groups holds
// samples chunk_b0 + [g*nb/ng, (g+1)*nb/ng) (nb = chunk_nb): contiguous ranges
// whose sizes differ by at most one.
struct Assign {
  int tile, g, ng;  // tile, group index, groups of the tile
  int first;        // list index of the tile's group 0 (its slots are first .. first+ng-1)
  int b0, nb;       // first sample, number of samples
};

__device__ __forceinline__ Assign assign_of(const Args& p, int j) {
  Assign a;
  const int q = p.gq, big = p.gr * (q + 1);
  if (j < big) {
    a.tile = j / (q + 1);
    a.g = j - a.tile * (q + 1);
    a.ng = q + 1;
    a.first = a.tile * (q + 1);
  } else {
    const int jj = j - big;
    a.tile = p.gr + jj / q;
    a.g = jj - (a.tile - p.gr) * q;
    a.ng = q;
    a.first = big + (a.tile - p.gr) * q;
  }
  const int nb = static_cast<int>(p.chunk_nb);
  const int lo = (a.g * nb) / a.ng, hi = ((a.g + 1) * nb) / a.ng;
  a.b0 = static_cast<int>(p.chunk_b0) + lo;
  a.nb = hi - lo;
  return a;
}

// Hardware workgroup -> list index: perm[] (host-made, see order_workgroups)
// when the grid has at most kPermMax workgroups, else the identity.
__device__ __forceinline__ int list_index(const Args& p, int hw) {
  return p.nwg <= kPermMax ? static_cast<int>(p.perm[hw]) : hw;
}

// out rows of a 128x128 tile staged in LDS as four 32-row quarters (fp32,
// row-major, 16 KB each): row r, column c at quarter r/32, (r%32)*128 + c.
__device__ __forceinline__ float* quarter(float* const (&q)[4], int i) {
  switch (i) {
    case 0: return q[0];
    case 1: return q[1];
    case 2: return q[2];
    default: return q[3];
  }
}
// The 8 staged floats [col, col+8) of a row (col a multiple of 8), as two
// 16-byte reads.  The 16 lanes reading one row take chunks 32 bytes apart, so
// the chunks of the row's upper half read their second half first: each read
// then covers all 64 banks once.
__device__ __forceinline__ void staged8(const float* row, int col, float (&v)[8]) {
  const bool up = (col & 64) != 0;
  const f32x4 a = *reinterpret_cast<const f32x4*>(row + col + (up ? 4 : 0));
  const f32x4 b = *reinterpret_cast<const f32x4*>(row + col + (up ? 0 : 4));
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = up ? b[e] : a[e];
    v[4 + e] = up ? a[e] : b[e];
  }
}
__device__ __forceinline__ float* staged_row(float* const (&q)[4], int r) {
  return quarter(q, r >> 5) + (r & 31) * BN;
}

// Noise for the 8 outputs (row m, columns n .. n+7 of a row of length N),
// unscaled; entries past N are zero.  Out of line: the Philox rounds are long,
// and an inlined copy per call site made the single-pass kernel hundreds of KB.
struct Z8 {
  float v[8];
};
__device__ __attribute__((noinline)) Z8 noise8_draw(NoiseSrc nz, int64_t N, int64_t m, int64_t n) {
  Z8 z = {};
  const bool whole = n + 8 <= N;
  if (whole && nz.z == nullptr && N % 4 == 0) {
    nz.run(m * N + n, z.v);
  } else if (whole && nz.z == nullptr) {
    nz.window(m * N + n, z.v);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (n + e < N) z.v[e] = nz.at(m * N + n + e);
  }
  return z;
}
// Only the last launch of a batch adds noise.
__device__ inline void noise8(const Args& p, int64_t m, int64_t n, float (&z)[8]) {
  const NoiseSrc nz = p.noise.resolved();  // a value copy: no address of the kernel argument is taken
  if (!p.chunk_last || !nz.on()) return;
  const Z8 d = noise8_draw(nz, p.N, m, n);
#pragma unroll
  for (int e = 0; e < 8; ++e) z[e] = d.v[e];
}

// Final values of 8 consecutive outputs (row m, columns n .. n+7 of the
// problem): the chunk carried from earlier launches is added; the result is
// carried on (not the last launch) or written as out_scale * v + noise_scale * z.
template <class OT>
__device__ inline void finish_chunk(const Args& p, int64_t m, int64_t n, float (&v)[8],
                                    const float (&z)[8]) {
  using S = typename OT::storage;
  const bool whole = n + 8 <= p.N;
  const bool cvec = whole && (p.N % 4 == 0);
  if (!p.chunk_first) {
    const float* src = p.chunk_acc + m * p.N + n;
    if (cvec) {
      const float4 c0 = reinterpret_cast<const float4*>(src)[0];
      const float4 c1 = reinterpret_cast<const float4*>(src)[1];
      v[0] += c0.x; v[1] += c0.y; v[2] += c0.z; v[3] += c0.w;
      v[4] += c1.x; v[5] += c1.y; v[6] += c1.z; v[7] += c1.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (n + e < p.N) v[e] += src[e];
    }
  }
  if (!p.chunk_last) {
    float* dst = p.chunk_acc + m * p.N + n;
    if (cvec) {
      reinterpret_cast<float4*>(dst)[0] = make_float4(v[0], v[1], v[2], v[3]);
      reinterpret_cast<float4*>(dst)[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (n + e < p.N) dst[e] = v[e];
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] *= p.out_scale;
  if (p.noise.on()) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] += p.noise_scale * z[e];
  }
  S* out = static_cast<S*>(p.out) + m * p.ldo + n;
  constexpr int E = 16 / sizeof(S);  // elements per 16-byte store
  const bool ovec = whole && reinterpret_cast<uintptr_t>(out) % 16 == 0;
  if (ovec) {
#pragma unroll
    for (int k = 0; k < 8 / E; ++k) {
      uint4 o;
      S* os = reinterpret_cast<S*>(&o);
#pragma unroll
      for (int e = 0; e < E; ++e) os[e] = OT::from_f32(v[k * E + e]);
      reinterpret_cast<uint4*>(out)[k] = o;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (n + e < p.N) out[e] = OT::from_f32(v[e]);
  }
}

// Exchange slot of list entry j: a 128x128 bf16 tile, row-major (the
// group's clipped sum, rounded once to bf16 for the exchange).
__device__ __forceinline__ const float* slot_of(const Args& p, int j) {
  return reinterpret_cast<const float*>(reinterpret_cast<const uint16_t*>(p.tile_acc) +
                                        int64_t(j) * (BM * BN));
}

// Rows [r0, r1) of the tile are taken as chunks of 8 outputs; a thread takes
// chunks c0, c0 + NT, ... kFinishChunks at a time.
constexpr int kFinishChunks = 4;
constexpr int kSlotBatch = 3;  // other groups' slots loaded together

// The noise of this thread's first kFinishChunks chunks of rows [r0, r1).
__device__ inline void noise_rows(const Args& p, int64_t m0, int64_t n0, int r0, int r1,
                                  float (&z)[kFinishChunks][8]) {
  const int nchunks = (r1 - r0) * (BN / 8);
#pragma unroll
  for (int k = 0; k < kFinishChunks; ++k) {
    const int c = threadIdx.x + k * NT;
    const int r = r0 + c / (BN / 8), col = (c % (BN / 8)) * 8;
    if (c < nchunks && m0 + r < p.M && n0 + col < p.N) noise8(p, m0 + r, n0 + col, z[k]);
  }
}

// Rows [r0, r1) of the tile: the staged sum of this group plus the slots of
// the tile's other groups (in group order; a fixed order per row), finished.
// The coherent slot loads of kSlotBatch groups and all kFinishChunks chunks
// are issued before any is used, so that they are in flight together.  zpre
// holds the noise of the first kFinishChunks chunks.
template <class OT>
__device__ inline void finish_rows(const Args& p, const Assign& as, int64_t m0, int64_t n0, int r0,
                                   int r1, float* const (&q4)[4], bool poisoned,
                                   const float (&zpre)[kFinishChunks][8]) {
  const int nchunks = (r1 - r0) * (BN / 8);
  for (int c0 = threadIdx.x; c0 < nchunks; c0 += NT * kFinishChunks) {
    float v[kFinishChunks][8];
#pragma unroll
    for (int k = 0; k < kFinishChunks; ++k) {
      const int c = c0 + k * NT;
      const int r = r0 + c / (BN / 8), col = (c % (BN / 8)) * 8;
      if (c < nchunks) {
        staged8(staged_row(q4, r), col, v[k]);
      }
    }
    for (int gb = 0; gb < as.ng; gb += kSlotBatch + 1) {
      // groups gb .. gb + kSlotBatch, this one's own left out
      u32x4 w[kSlotBatch + 1][kFinishChunks];
#pragma unroll
      for (int s = 0; s <= kSlotBatch; ++s) {
        const int gg = gb + s;
        if (gg >= as.ng || gg == as.g) continue;
        const CoherentSpan sl(slot_of(p, as.first + gg), BM * BN * 2);
#pragma unroll
        for (int k = 0; k < kFinishChunks; ++k) {
          const int c = c0 + k * NT;
          const int r = r0 + c / (BN / 8), col = (c % (BN / 8)) * 8;
          // chunks past the range read inside the slot (c < 2048) and are unused
          w[s][k] = __builtin_bit_cast(
              u32x4, sl.load4(static_cast<uint32_t>(((r * BN + col) * 2) & (BM * BN * 2 - 1))));
        }
      }
#pragma unroll
      for (int s = 0; s <= kSlotBatch; ++s) {
        const int gg = gb + s;
        if (gg >= as.ng || gg == as.g) continue;
#pragma unroll
        for (int k = 0; k < kFinishChunks; ++k)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[k][2 * e] += __uint_as_float(w[s][k][e] << 16);
            v[k][2 * e + 1] += __uint_as_float(w[s][k][e] & 0xffff0000u);
          }
      }
    }
    const bool first = c0 == static_cast<int>(threadIdx.x);
#pragma unroll
    for (int k = 0; k < kFinishChunks; ++k) {
      const int c = c0 + k * NT;
      if (c >= nchunks) continue;
      const int r = r0 + c / (BN / 8), col = (c % (BN / 8)) * 8;
      const int64_t m = m0 + r, n = n0 + col;
      if (m >= p.M || n >= p.N) continue;
      if (poisoned) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[k][e] = __builtin_nanf("");
      }
      float z[8] = {};
      if (first) {
#pragma unroll
        for (int e = 0; e < 8; ++e) z[e] = zpre[k][e];
      } else {
        noise8(p, m, n, z);
      }
      finish_chunk<OT>(p, m, n, v[k], z);
    }
  }
}

// List-index bit sets of the split products (Args::owner_mask / helper_mask).
__device__ __forceinline__ bool mask_has(const uint32_t* m, int j) {
  return (m[j >> 5] >> (j & 31)) & 1u;
}
// Entries of the set below j.
__device__ inline int mask_rank(const uint32_t* m, int j) {
  int r = 0;
  for (int w = 0; w < (j >> 5); ++w) r += __builtin_popcount(m[w]);
  return r + __builtin_popcount(m[j >> 5] & ((1u << (j & 31)) - 1u));
}
// The r-th entry of the set, or -1.
__device__ inline int mask_select(const uint32_t* m, int r) {
  for (int w = 0; w < kPermMax / 32; ++w) {
    uint32_t x = m[w];
    const int c = __builtin_popcount(x);
    if (r < c) {
      for (; r > 0; --r) x &= x - 1u;  // drop the r lowest set bits
      return w * 32 + __builtin_ctz(x);
    }
    r -= c;
  }
  return -1;
}

// Hand-over of a split product through an exchange slot: each thread's 64
// accumulators as 32 bf16 pairs (RNE), in 16-byte chunks q at byte
// (q * NT + thread) * 16, agent-coherent.
__device__ inline void hand_over(const float* slot, const f32x16 (&acc)[2][2]) {
  const CoherentSpan sp(slot, BM * BN * 2);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int q = (i * 2 + j) * 2 + half;
        u32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 8 * half + 2 * e;
          w[e] = BF16::pack2(acc[i][j][r], acc[i][j][r + 1]);
        }
        sp.store4(static_cast<uint32_t>((q * NT + threadIdx.x) * 16), __builtin_bit_cast(f32x4, w));
      }
}
// acc += the product handed over in the slot.
__device__ inline void take_over(const float* slot, f32x16 (&acc)[2][2]) {
  const CoherentSpan sp(slot, BM * BN * 2);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int q = (i * 2 + j) * 2 + half;
        const u32x4 w = __builtin_bit_cast(
            u32x4, sp.load4(static_cast<uint32_t>((q * NT + threadIdx.x) * 16)));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 8 * half + 2 * e;
          acc[i][j][r] += __uint_as_float(w[e] << 16);
          acc[i][j][r + 1] += __uint_as_float(w[e] & 0xffff0000u);
        }
      }
}

// Workgroups of the grid run their nb products, keeping the finished ones
// packed in registers and the last one live in its accumulators; each
// product's sum of squares goes to partials[sample, tile].  After the grid
// barrier every workgroup knows the norms of its samples and forms
// sum_b c_b G_b for its tile (fixed order: deterministic).  The groups of a
// tile then exchange their sums: group g publishes the rows the other groups
// finish, waits for the tile's other groups, and finishes rows
// [g*128/ng, (g+1)*128/ng) itself (output, or the running sum carried to the
// next launch in chunk_acc).
// BOP 1 / 2: also the bias of operand a / b (bias_finish): every product's
// column sums and squares are taken from its fragments and stored at the
// product's end; after the last launch's grid barrier and the row finish,
// workgroups [0, ceil(bias_len / kBiasCols)) finish the bias.  Split products
// are not used then (the host sets split_k1 = 0).
constexpr int kStages = 2;  // LDS ring depth of the single-pass kernel (64-deep k-tiles)

template <class DT, int U, int BOP = 0>
__global__ __launch_bounds__(NT, 2) void wgrad_group_kernel(Args p) {
  using G = dma::Geom<BM, BN, 64>;
  static_assert(kStages * G::STAGE == BM * BN * 4, "the output staging reuses the ring");
  static_assert(U <= NT / kWave, "one wavefront per held sample forms its factor");
  __shared__ __attribute__((aligned(16))) char st0[G::STAGE];
  __shared__ __attribute__((aligned(16))) char st1[G::STAGE];
  __shared__ float red[NT / kWave];
  __shared__ float fac[U];
  __shared__ int flag;
  __shared__ float bcol[BOP != 0 ? BM : 1];  // a product's folded bias column sums
  __shared__ float bred[NT / kWave];
  // every product's partials (sum of squares; the bias's column sums and sum
  // of squares) wait here until the k-loop is over: a store issued inside the
  // loop would make the ring's vmcnt waits wait for the next k-tile's loads
  __shared__ float wsq[U];
  __shared__ float bpend[BOP != 0 ? U * BM : 1];
  __shared__ float bsqp[U];
  const dma::Stages stages{{(FDP_LDS char*)(st0), (FDP_LDS char*)(st1),
                            (FDP_LDS char*)(st0), (FDP_LDS char*)(st1)}};
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int tiles = p.tiles_m * p.tiles_n;
  const int me = list_index(p, blockIdx.x);
  const Assign as = assign_of(p, me);
  const int nb = as.nb;
  const int nk = static_cast<int>((p.K + G::BK - 1) / G::BK);
  dma::FragOffsets<G> fo;
  fo.init(wm, wn);
  const uint64_t t_begin = wall_clock64();
  // this launch's tag, in thread 0 (the only thread taking part in the
  // waits); its first use is far away, so the load's latency is hidden, and
  // grid_arrive() completes it (vmcnt(0), fence) before this workgroup arrives
  unsigned tag = 0;
  if (threadIdx.x == 0)
    tag = __hip_atomic_load(p.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;

  // ---- phase 1: the nb products run as one stream of nb*nk k-tiles through
  // the LDS ring, so that the next unit's first k-tiles load while this
  // unit's last ones multiply and its norm is taken.
  const uint16_t* pa = static_cast<const uint16_t*>(p.a);
  const uint16_t* pb = static_cast<const uint16_t*>(p.b);
  Held<true> held[U > 1 ? U - 1 : 1];
  // Split product (see pair_products): an owner's last unit covers k-tiles
  // [0, k1) of its last sample; a helper first runs k-tiles [k1, nk) of its
  // owner's last sample and tile, then its own units.
  const int k1 = p.split_k1;
  int role = 0, pair = 0, owner = me;  // role 1: owner, 2: helper
  if (k1 > 0 && nb > 0) {
    if (mask_has(p.owner_mask, me)) {
      role = 1;
      pair = mask_rank(p.owner_mask, me);
    } else if (mask_has(p.helper_mask, me)) {
      pair = mask_rank(p.helper_mask, me);
      owner = mask_select(p.owner_mask, pair);
      role = owner >= 0 ? 2 : 0;
      if (owner < 0) owner = me;
    }
  }
  auto unit_nk = [&](int u) { return role == 1 && u == nb - 1 ? k1 : nk; };
  const int nq = role == 1 ? (nb - 1) * nk + k1 : nb * nk;
  dma::Job<G> job;  // loads of k-tile ik of unit iu, the next one to issue
  int iu = 0, ik = 0;
  int64_t m0, n0;
  tile_coords(p, as.tile, m0, n0);
  // bias: the tile's index along the other axis; of the two waves sharing a
  // row (column) of fragments, this one sums fragment bws: its tile columns
  // from bcl (bias_frag)
  const int bother = BOP == 1 ? static_cast<int>(n0 / BN) : static_cast<int>(m0 / BM);
  const int bws = BOP == 1 ? (wave & 1) : (wave >> 1);
  const int bcl = (BOP == 1 ? wm : wn) + 32 * bws;
  const int blim = bias_limit(p.bias_len, BOP == 1 ? m0 : n0);
  float bcs[1] = {0.f}, bsq = 0.f;
  (void)bother;
  (void)bws;
  (void)bcl;
  (void)blim;
  // rows [r0, r1) of the tile are finished by this group; their noise (VALU
  // work independent of the data) is drawn ahead into zpre: by workgroups with
  // fewer products than the most loaded ones while they wait at the grid
  // barrier, by the others while the tile's groups publish
  const int r0 = (as.g * BM) / as.ng, r1 = ((as.g + 1) * BM) / as.ng;
  float zpre[kFinishChunks][8] = {};
  const bool early = nb < U;
  // The more loaded workgroup of a CU issues first (wave priority), so that
  // the two of a CU finish their products together instead of the more loaded
  // one running its last stretch alone.
  const bool loaded = k1 > 0 ? role != 0 : nb == U;
  if (loaded) __builtin_amdgcn_s_setprio(2);
  f32x16 acc[2][2];
  zero(acc);
  if (role == 2) {
    // helper: k-tiles [k1, nk) of the owner's last product first, handed over
    // through the owner's exchange slot, then the hand-over flag
    const Assign oa = assign_of(p, owner);
    int64_t om0, on0;
    tile_coords(p, oa.tile, om0, on0);
    const int64_t ob = oa.b0 + oa.nb - 1;
    const int64_t kr = int64_t(k1) * G::BK;
    job.init(pa + ob * p.sab + kr * p.lda, p.lda, pb + ob * p.sbb + kr * p.ldb, p.ldb, p.K - kr,
             om0, on0);
    dma::gemm<DT, G, kStages>(job, nk - k1, fo, stages, acc);
    hand_over(slot_of(p, owner), acc);
    zero(acc);
    wait_stores();  // (the ring's first wait below would drain them anyway)
    __syncthreads();
    if (threadIdx.x == 0)
      __hip_atomic_store(p.pair_flag + pair, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (nq > 0)
    job.init(pa + as.b0 * p.sab, p.lda, pb + as.b0 * p.sbb, p.ldb,
             role == 1 && nb == 1 ? int64_t(k1) * G::BK : p.K, m0, n0);
  auto issue_next = [&](FDP_LDS char* stage) {
    job.issue(stage, ik);
    if (++ik == unit_nk(iu)) {
      ik = 0;
      if (++iu < nb) {
        const int64_t b = as.b0 + iu;
        job.retarget(pa + b * p.sab, p.lda, pb + b * p.sbb, p.ldb,
                     role == 1 && iu == nb - 1 ? int64_t(k1) * G::BK : p.K);
      }
    }
  };
  dma::wait_vm<0>();
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s)
    if (s < nq) issue_next(stages.get(s));
  int cu = 0, ck = 0;  // unit / k-tile being multiplied
  for (int base = 0; base < nq; base += kStages) {
#pragma unroll
    for (int s = 0; s < kStages; ++s) {
      const int q = base + s;
      if (q < nq) {
        const int ahead = nq - 1 - q;
        dma::wait_tiles<G::LOADS>(ahead < kStages - 2 ? ahead : kStages - 2);
        dma::barrier();
        if (q + kStages - 1 < nq) issue_next(stages.get((s + kStages - 1) % kStages));
        if constexpr (BOP != 0) {
          const bool counted = ck % p.bias_P == bother;
          dma::compute_stage_f<DT, G>(stages.get(s), fo, acc, [&](int, const dma::Frags<G>& f) {
            if (counted) {
              const uint4 fr = BOP == 1 ? (bws == 0 ? f.a[0] : f.a[1]) : (bws == 0 ? f.b[0] : f.b[1]);
              bias_frag<DT>(fr, bcs[0], bsq, bcl + (lane & 31), blim);
            }
          });
        } else {
          dma::compute_stage<DT, G>(stages.get(s), fo, acc);
        }
        if (++ck == unit_nk(cu)) {
          {
            const int own = cu;
            // Rows/columns past M/N may hold the next row's values: leave
            // them out of the norm.
            float sq = 0.f;
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
              for (int c = 0; c < 2; ++c) {
                const bool ncol = n0 + acc_col(wn, c, lane) < p.N;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                  const bool in = ncol && (m0 + acc_row(wm, a, lane, r) < p.M);
                  sq += in ? acc[a][c][r] * acc[a][c][r] : 0.f;
                }
              }
            sq = wave_sum(sq);
            if (lane == 0) red[wave] = sq;
            if constexpr (BOP != 0) bias_fold<1>(bcs, bsq, bcol, bred, bcl);
            __syncthreads();
            if (threadIdx.x == 0) wsq[own] = (red[0] + red[1]) + (red[2] + red[3]);
            if constexpr (BOP != 0) bias_park<BM>(bcol, bred, bpend + own * BM, bsqp + own);
            if (own + 1 < nb) {  // park it and start the next product
#pragma unroll
              for (int j = 0; j < U - 1; ++j)
                if (j == own) held[j].put(acc);
              zero(acc);
              if (role == 1 && own + 2 == nb) {
                // owner: the last product starts from the helper's share (its
                // load latency overlaps that of the product's first k-tiles)
                if (threadIdx.x == 0) {
                  for (unsigned spins = 0;; ++spins) {
                    if (spins >= p.spin_limit) {
                      expire(p.err, p.poison, tag);  // every workgroup's results are poisoned
                      break;
                    }
                    if (__hip_atomic_load(p.pair_flag + pair, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT) == tag)
                      break;
                    __builtin_amdgcn_s_sleep(kPollSleep);
                  }
                }
                __syncthreads();
                take_over(slot_of(p, me), acc);
              }
            }
          }
          ck = 0;
          ++cu;
        }
      }
    }
  }
  dma::barrier();  // every wave is done reading the ring (and the parked partials are written)
  if (threadIdx.x < nb)
    st_coherent(p.partials + (as.b0 + threadIdx.x) * tiles + as.tile, wsq[threadIdx.x]);
  if constexpr (BOP != 0) {
    for (int u = 0; u < nb; ++u)
      bias_store<BM>(p, bpend + u * BM, bsqp[u], as.b0 + u, as.tile, tiles, BOP == 1 ? m0 : n0,
                     bother);
  }

  // The tile's exchange ticket starts at zero in every launch: group 0 clears
  // it before the grid barrier, every ticket is taken after it.  (A ticket
  // word may hold another problem's data: workspace layouts differ by shape.)
  if (threadIdx.x == 0 && as.ng > 1 && as.g == 0)
    __hip_atomic_store(p.tile_turn + as.tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // A wait that expired (only possible when the grid was not resident at once)
  // poisons this workgroup's results with NaN rather than leave them silently
  // wrong; the status word reports it.
  // Workgroups with fewer products than the launch's most loaded ones wait
  // quietly for about 60% of the time those need for the rest of theirs
  // (measured on this workgroup's own products; a workgroup left alone on its
  // CU runs its last product faster than two sharing the CU, and a late wake-up
  // delays this tile's exchange).
  uint64_t quiet = 0;
  {
    // in half products: the most loaded workgroups' work and this one's
    const int most = 2 * U - (k1 > 0 ? 1 : 0), mine = 2 * nb + (role == 1 ? -1 : role == 2 ? 1 : 0);
    if (nb > 0 && mine < most) {
      const uint64_t now = wall_clock64();
      quiet = now + (now - t_begin) * uint64_t(3 * (most - mine)) / uint64_t(5 * mine);
    }
  }
  if (loaded) __builtin_amdgcn_s_setprio(0);
  const unsigned arrival = grid_arrive(p.bar);
  if (early) noise_rows(p, m0, n0, r0, r1, zpre);
  bool poisoned = grid_wait(p.bar, unsigned(p.nwg), arrival, p.err, p.epoch, p.poison, tag,
                            p.spin_limit, &flag, quiet);

  // ---- clip factors of this workgroup's samples: wavefront i sums the
  // partials of sample b0 + i in a fixed order
  {
    float C = p.C, clamp = p.clamp;
    if (p.clip_args_dev != nullptr) {
      C = p.clip_args_dev[0];
      clamp = p.clip_args_dev[1];
    }
    if (wave < nb) {
      const float* part = p.partials + int64_t(as.b0 + wave) * tiles;
      float s = 0.f;
      for (int t = lane; t < tiles; t += kWave) s += ld_coherent(part + t);
      s = wave_sum(s);
      if (lane == 0) {
        const float n = poisoned ? __builtin_nanf("") : sqrtf(s);
        const float cf = poisoned ? n : clip_factor(n, C, clamp);
        fac[wave] = cf;
        if (as.tile == 0) {  // one writer per sample
          if (p.norms_out) p.norms_out[as.b0 + wave] = n;
          if (p.factors_out) p.factors_out[as.b0 + wave] = cf;
        }
      }
    }
    __syncthreads();
  }

  // ---- phase 2: sum_b c_b G_b formed in place in the accumulators as
  // c_last G_last + c_0 G_0 + c_1 G_1 + ... (a fixed order: deterministic)
  if (nb > 0) {
    const float cl = fac[nb - 1];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][c][r] *= cl;
  } else {
    zero(acc);
  }
#pragma unroll
  for (int j = 0; j < U - 1; ++j)
    if (j < nb - 1) held[j].add_to(acc, fac[j]);

  // stage the group's sum in LDS, row-major (the ring is free)
  float* const q4[4] = {reinterpret_cast<float*>(st0), reinterpret_cast<float*>(st0) + 4096,
                        reinterpret_cast<float*>(st1), reinterpret_cast<float*>(st1) + 4096};
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    float* qd = quarter(q4, wm / 32 + a);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) qd[acc_row(0, 0, lane, r) * BN + acc_col(wn, c, lane)] = acc[a][c][r];
  }
  __syncthreads();
  if (as.ng > 1) {
    // publish the rows the other groups finish (row-major slot), then wait
    // until every group of the tile has published
    const uint64_t t_pub = wall_clock64();
    const CoherentSpan mine(slot_of(p, as.first + as.g), BM * BN * 2);
    for (int c = threadIdx.x; c < BM * (BN / 8); c += NT) {
      const int r = c / (BN / 8), col = (c % (BN / 8)) * 8;
      if (r >= r0 && r < r1) continue;
      float src[8];
      staged8(staged_row(q4, r), col, src);
      u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w[e] = BF16::pack2(src[2 * e], src[2 * e + 1]);
      mine.store4(static_cast<uint32_t>((r * BN + col) * 2), __builtin_bit_cast(f32x4, w));
    }
    wait_stores();
    __syncthreads();
    uint64_t quiet_until = 0;
    if (threadIdx.x == 0) {
      __hip_atomic_fetch_add(p.tile_turn + as.tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // the tile's other groups started publishing together with this one:
      // stay off the memory pipeline for a fraction of this group's own time
      const uint64_t now = wall_clock64();
      quiet_until = now + (now - t_pub) / 2;
    }
    if (!early) noise_rows(p, m0, n0, r0, r1, zpre);
    if (threadIdx.x == 0) {
      while (wall_clock64() < quiet_until) __builtin_amdgcn_s_sleep(8);
      int bad = 0;
      for (unsigned spins = 0;; ++spins) {
        if (spins >= p.spin_limit) {
          expire(p.err, p.poison, tag);
          bad = 1;
          break;
        }
        if (__hip_atomic_load(p.tile_turn + as.tile, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >=
            unsigned(as.ng))
          break;
        __builtin_amdgcn_s_sleep(kPollSleep);
      }
      flag = bad;
    }
    __syncthreads();
    poisoned = poisoned || flag != 0;
  }
  if (!early && as.ng == 1) noise_rows(p, m0, n0, r0, r1, zpre);
  // The control words are zero again: the grid barrier resets its counter, and
  // group 0 of each tile clears the tile's ticket before that barrier.
  if (p.out_dtype == FDP_BF16) finish_rows<BF16>(p, as, m0, n0, r0, r1, q4, poisoned, zpre);
  else if (p.out_dtype == FDP_F16) finish_rows<F16>(p, as, m0, n0, r0, r1, q4, poisoned, zpre);
  else finish_rows<F32>(p, as, m0, n0, r0, r1, q4, poisoned, zpre);
  if constexpr (BOP != 0) {
    // every sample's partials are visible: this launch's since the grid
    // barrier, earlier launches' by stream order
    if (p.chunk_last && int64_t(blockIdx.x) * kBiasCols < p.bias_len) {
      __syncthreads();  // the staged rows in the ring are read
      bias_finish(p, tiles, blockIdx.x, p.nwg, poisoned, *reinterpret_cast<BiasSmem*>(st0));
    }
  }
}

// Clears the barrier / ticket words at the head of the workspace.
template <int kUnused = 0>
__global__ __launch_bounds__(NT) void clear_words_kernel(unsigned* p, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * NT + threadIdx.x; i < n; i += int64_t(gridDim.x) * NT)
    p[i] = 0u;
}

// ---------------------------------------------------------- single-pass launch
using KernelFn = void (*)(Args);
// Control words at the head of the workspace: word 0 the status word (sticky,
// for the host), word 1 the grid-barrier counter (zero between launches),
// word 2 the launch epoch, word 3 the poison tag, words [kPairFlag0,
// kPairFlag0 + kPairMax) the split-product flags (tagged).  A zero-filled head
// is a valid start; every launch leaves it valid.
constexpr size_t kWsHead = 2048;
constexpr int kPairFlag0 = 64;
static_assert((kPairFlag0 + kPairMax) * sizeof(unsigned) <= kWsHead, "control words");
// Words [kGroupWord0, kGroupWord0 + kGroupMax): the paired wide kernel's
// per-tile counters (zero between launches).
constexpr int kGroupWord0 = kPairFlag0 + kPairMax;
constexpr int kGroupMax = static_cast<int>(kWsHead / sizeof(unsigned)) - kGroupWord0;
constexpr int kGroupUnits = 4;    // samples held by one workgroup at most

// Single-pass schedule for B samples over `tiles` 128x128 tiles on `slots`
// co-resident workgroups (2 per CU).  A launch covers `chunk` samples (the
// last one fewer) with at most kGroupUnits samples per workgroup; its grid has
// min(slots, tiles * chunk) workgroups.  chunk == 0: more tiles than slots,
// no single pass (the streamed two-pass schedule is used).
struct GroupPlan {
  int64_t chunk;  // samples per launch
  int max_nwg;    // workgroups of the largest launch
};
inline GroupPlan group_plan(int64_t B, int tiles, int slots) {
  GroupPlan g{};
  if (tiles > slots) return g;
  const int64_t gcap = slots / tiles;  // groups per tile that fit the grid
  g.chunk = gcap * kGroupUnits < B ? gcap * kGroupUnits : B;
  const int64_t w = int64_t(tiles) * g.chunk;
  g.max_nwg = static_cast<int>(w < slots ? w : slots);
  return g;
}

// Grid of one launch over nb samples: W workgroups, gq groups per tile (gr
// tiles have one more), at most `units` samples per workgroup.
struct LaunchShape {
  int nwg, gq, gr, units;
};
inline LaunchShape launch_shape(int64_t nb, int tiles, int slots) {
  LaunchShape l{};
  const int64_t w = int64_t(tiles) * nb < slots ? int64_t(tiles) * nb : slots;
  l.nwg = static_cast<int>(w);
  l.gq = static_cast<int>(w / tiles);
  l.gr = static_cast<int>(w % tiles);
  l.units = static_cast<int>((nb + l.gq - 1) / l.gq);
  return l;
}

// Hardware workgroup -> work list index.  Workgroups are dealt round-robin
// to the 8 XCDs, and on an otherwise idle device workgroups w and w + CUs
// share a CU.  The entries with the most samples ("heavy") and the others are
// each sorted by (first sample, tile) and cut into 8 equal contiguous shares,
// one per XCD: every XCD gets the same work, and its workgroups step through
// the same samples over neighbouring (band-ordered) tiles at the same time, so
// they share operand tiles in that XCD's L2.  Within an XCD the heavy entries
// come first, so that they share their CUs (k and k + CUs/8) with light ones.
// The order only affects speed.
inline void order_workgroups(const Args& c, int cus, uint16_t* perm) {
  const int W = c.nwg;
  for (int i = 0; i < W && i < kPermMax; ++i) perm[i] = static_cast<uint16_t>(i);
  if (W > kPermMax || W % kXcds != 0 || cus % kXcds != 0) return;
  const int n = W / kXcds;
  const int nb = static_cast<int>(c.chunk_nb), q = c.gq, big = c.gr * (q + 1);
  int key[kPermMax], units[kPermMax], heavy[kPermMax], light[kPermMax];
  int umax = 0;
  for (int j = 0; j < W; ++j) {
    int tile, g, ng;
    if (j < big) {
      ng = q + 1;
      tile = j / ng;
      g = j % ng;
    } else {
      ng = q;
      tile = c.gr + (j - big) / q;
      g = (j - big) % q;
    }
    const int lo = (g * nb) / ng;
    units[j] = ((g + 1) * nb) / ng - lo;
    key[j] = lo * (c.tiles_m * c.tiles_n) + tile;
    umax = units[j] > umax ? units[j] : umax;
  }
  int nh = 0, nl = 0;
  for (int j = 0; j < W; ++j) {
    if (units[j] == umax) heavy[nh++] = j;
    else light[nl++] = j;
  }
  // insertion sorts by key (W <= kPermMax; on the host, once per launch)
  auto sort = [&](int* v, int len) {
    for (int i = 1; i < len; ++i) {
      const int x = v[i];
      int k = i - 1;
      while (k >= 0 && key[v[k]] > key[x]) {
        v[k + 1] = v[k];
        --k;
      }
      v[k + 1] = x;
    }
  };
  sort(heavy, nh);
  sort(light, nl);
  for (int x = 0; x < kXcds; ++x) {
    const int h0 = (x * nh) / kXcds, h1 = ((x + 1) * nh) / kXcds;
    const int l0 = (x * nl) / kXcds, l1 = ((x + 1) * nl) / kXcds;
    // an XCD's share is n entries when nh and nl split evenly; otherwise the
    // shares are rebalanced below so that every XCD has exactly n
    int k = 0;
    for (int i = h0; i < h1 && k < n; ++i) perm[x + kXcds * k++] = static_cast<uint16_t>(heavy[i]);
    for (int i = l0; i < l1 && k < n; ++i) perm[x + kXcds * k++] = static_cast<uint16_t>(light[i]);
    if (k != n) {  // uneven split: fall back to the plain sorted order
      for (int i = 0; i < W && i < kPermMax; ++i) perm[i] = static_cast<uint16_t>(i);
      return;
    }
  }
}

// Split products.  With W = 2*CUs workgroups and entries of two sizes,
// order_workgroups puts each most-loaded entry ("heavy", umax products) on a CU
// of its own beside a lighter one, and the remaining lighter entries two to a
// CU.  A CU with a heavy entry then carries one product more than a CU with
// two light ones, and runs that product alone at the lone-workgroup rate.  Each
// heavy entry ("owner") therefore contracts its last product over only the
// first split_k1 k-tiles; the first lighter entry of a light-light CU
// ("helper") contracts the rest, before its own products, and hands the
// partial product over as bf16 through the owner's exchange slot.  Every CU
// then carries umax + umin - 1/2 products.  The r-th owner in list order
// pairs with the r-th helper.  No split when the counts differ, the grid is
// not 2*CUs, or there are fewer than two k-tiles.
inline void pair_products(Args& c, int cus) {
  for (int w = 0; w < kPermMax / 32; ++w) c.owner_mask[w] = c.helper_mask[w] = 0u;
  c.split_k1 = 0;
  const int W = c.nwg;
  const int nk = static_cast<int>((c.K + 63) / 64);
  if (W != 2 * cus || W > kPermMax || nk < 2) return;
  const int nb = static_cast<int>(c.chunk_nb), q = c.gq, big = c.gr * (q + 1);
  auto units_of = [&](int j) {
    int g, ng;
    if (j < big) {
      ng = q + 1;
      g = j % ng;
    } else {
      ng = q;
      g = (j - big) % q;
    }
    return ((g + 1) * nb) / ng - (g * nb) / ng;
  };
  int umax = 0, umin = 1 << 30;
  for (int j = 0; j < W; ++j) {
    const int u = units_of(j);
    umax = u > umax ? u : umax;
    umin = u < umin ? u : umin;
  }
  if (umax == umin || umin < 1) return;
  int owners = 0, helpers = 0;
  for (int j = 0; j < W; ++j)
    if (units_of(j) == umax) ++owners;
  for (int h = 0; h < cus; ++h)
    if (units_of(c.perm[h]) < umax && units_of(c.perm[h + cus]) < umax) ++helpers;
  if (owners == 0 || owners != helpers || owners > kPairMax) return;
  for (int j = 0; j < W; ++j)
    if (units_of(j) == umax) c.owner_mask[j / 32] |= 1u << (j % 32);
  for (int h = 0; h < cus; ++h)
    if (units_of(c.perm[h]) < umax && units_of(c.perm[h + cus]) < umax) {
      const int j = c.perm[h];
      c.helper_mask[j / 32] |= 1u << (j % 32);
    }
  c.split_k1 = nk / 2;
}

// Host-made part of a launch's Args (order_workgroups, pair_products).
struct WorkMap {
  uint16_t perm[kPermMax];
  uint32_t owner_mask[kPermMax / 32];
  uint32_t helper_mask[kPermMax / 32];
  int split_k1;
};
using WorkMapKey = std::tuple<int, int, int64_t, int64_t, int>;
inline host::ShapeCache<WorkMapKey, WorkMap>& work_map_cache() {
  static host::ShapeCache<WorkMapKey, WorkMap> c;
  return c;
}

// `plain`: ordinary dispatch instead of a cooperative launch (the caller
// guarantees that nothing else occupies the device during the call, so the
// grid, sized to the computed occupancy, is resident at once).  `clean`: the
// control words are already zero (every launch of the kernel leaves them so),
// which makes the clearing kernel unnecessary.
template <class DT, int BOP = 0>
hipError_t try_grouped(Args a, int cus, bool plain, bool clean, hipStream_t s) {
  const int tiles = a.tiles_m * a.tiles_n;
  if (!fits_record(a.K, a.lda) || !fits_record(a.K, a.ldb)) return hipErrorNotSupported;
  const GroupPlan gp = group_plan(a.B, tiles, 2 * cus);
  if (gp.chunk == 0) return hipErrorNotSupported;
  KernelFn grouped[kGroupUnits] = {&wgrad_group_kernel<DT, 1, BOP>, &wgrad_group_kernel<DT, 2, BOP>,
                                   &wgrad_group_kernel<DT, 3, BOP>, &wgrad_group_kernel<DT, 4, BOP>};
  const int64_t words = int64_t(kWsHead / sizeof(unsigned));
  for (int64_t b0 = 0; b0 < a.B; b0 += gp.chunk) {
    Args c = a;
    c.chunk_b0 = b0;
    c.chunk_nb = a.B - b0 < gp.chunk ? a.B - b0 : gp.chunk;
    const LaunchShape ls = launch_shape(c.chunk_nb, tiles, 2 * cus);
    c.nwg = ls.nwg;
    c.gq = ls.gq;
    c.gr = ls.gr;
    c.chunk_first = b0 == 0;
    c.chunk_last = b0 + c.chunk_nb >= a.B;
    // The work map depends only on the tile grid, the launch's samples, the
    // number of k-tiles and the CU count: cached per shape.
    const WorkMap wm = work_map_cache().get(
        std::make_tuple(a.tiles_m, a.tiles_n, c.chunk_nb, (c.K + 63) / 64, cus), [&] {
          WorkMap w{};
          order_workgroups(c, cus, w.perm);
          std::memcpy(c.perm, w.perm, sizeof(w.perm));
          pair_products(c, cus);
          std::memcpy(w.owner_mask, c.owner_mask, sizeof(w.owner_mask));
          std::memcpy(w.helper_mask, c.helper_mask, sizeof(w.helper_mask));
          w.split_k1 = c.split_k1;
          return w;
        });
    std::memcpy(c.perm, wm.perm, sizeof(wm.perm));
    std::memcpy(c.owner_mask, wm.owner_mask, sizeof(wm.owner_mask));
    std::memcpy(c.helper_mask, wm.helper_mask, sizeof(wm.helper_mask));
    c.split_k1 = wm.split_k1;
    if (BOP != 0) {  // the bias counts k-tiles per (sample, tile): no split products
      c.split_k1 = 0;
      for (int w = 0; w < kPermMax / 32; ++w) c.owner_mask[w] = c.helper_mask[w] = 0u;
    }
    KernelFn fn = grouped[ls.units - 1];
    if (host::occupancy(reinterpret_cast<const void*>(fn), NT, 0) < 2) return hipErrorNotSupported;
    if (b0 == 0 && !clean)
      hipLaunchKernelGGL(clear_words_kernel<0>,
                         dim3(static_cast<unsigned>((words + NT - 1) / NT)), dim3(NT), 0, s,
                         reinterpret_cast<unsigned*>(a.err), words);
    void* params[] = {&c};
    const hipError_t e =
        plain ? hipLaunchKernel(reinterpret_cast<const void*>(fn), dim3(c.nwg), dim3(NT), params, 0, s)
              : hipLaunchCooperativeKernel(reinterpret_cast<const void*>(fn), dim3(c.nwg),
                                           dim3(NT), params, 0, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// Per-dtype launchers (wgrad_group_{bf16,f16}.hip; with the bias of operand
// a.bias_op, wgrad_group_bias_{bf16,f16}.hip).
hipError_t launch_grouped_bf16(Args a, int cus, bool plain, bool clean, hipStream_t s);
hipError_t launch_grouped_f16(Args a, int cus, bool plain, bool clean, hipStream_t s);
hipError_t launch_grouped_bias_bf16(Args a, int cus, bool plain, bool clean, hipStream_t s);
hipError_t launch_grouped_bias_f16(Args a, int cus, bool plain, bool clean, hipStream_t s);

}  // namespace wg
}  // namespace fdp
