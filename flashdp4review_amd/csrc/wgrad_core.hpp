// Shared pieces of the clipped per-sample weight-gradient kernels: operand
// loaders and MFMA tile cores for gfx950, and the single-pass cooperative kernel
// template (instantiated per dtype in wgrad_fused_*.hip, launched from
// wgrad_clip.hip).  See wgrad_clip.hip for the algorithm.
#pragma once

#include "fdp_common.hpp"
#include "gemm_dma.hpp"

namespace fdp {
namespace wg {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int NT = 256;

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
  unsigned* done;         // workgroups finished (the last one re-zeroes bar / done)
  unsigned* tile_turn;    // [tiles] hand-over tickets for tiles shared by workgroups
  float* tile_acc;        // [tiles, BM*BN] fp32 running sums of shared tiles
  int* err;               // set when a bounded wait gives up
  unsigned spin_limit;    // polls before a grid wait gives up
  float C, clamp;
  const float* clip_args_dev;
  float* norms_out;       // optional [B]
  float* factors_out;     // optional [B]
  // single-pass kernel: this launch covers samples [chunk_b0, chunk_b0+chunk_nb)
  int64_t chunk_b0, chunk_nb;
  int chunk_first, chunk_last;
  float* chunk_acc;       // [M, N] fp32 running sum carried between chunks
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
constexpr int kXcds = 8;


// All workgroups of the (co-resident) grid arrive before any leaves.  Returns
// (in every thread) whether this workgroup's results must be poisoned: its own
// wait expired, or an earlier workgroup's did (that one set *err before this
// one could arrive).
__device__ inline bool grid_barrier(unsigned* bar, unsigned n, int* err, unsigned limit,
                                    int* flag) {
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned spins = 0;
    int bad = 0;
    while (__hip_atomic_load(bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < n) {
      __builtin_amdgcn_s_sleep(1);
      if (++spins > limit) {
        atomicOr(err, 1);
        bad = 1;
        break;
      }
    }
    if (!bad) bad = __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
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
struct Held<true> {  // 64 fp32 accumulators -> 32 bf16 pairs parked in AGPRs
  uint32_t v[2][2][8];
  __device__ __forceinline__ void put(const f32x16 (&acc)[2][2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const uint32_t w = uint32_t(BF16::from_f32(acc[i][j][2 * q])) |
                             (uint32_t(BF16::from_f32(acc[i][j][2 * q + 1])) << 16);
          asm volatile("v_accvgpr_write_b32 %0, %1" : "=a"(v[i][j][q]) : "v"(w));
        }
  }
  __device__ __forceinline__ void add_to(f32x16 (&tot)[2][2], float c) const {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          uint32_t w;
          asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(w) : "a"(v[i][j][q]));
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

// Tile-local fp32 buffer access in the accumulator layout (coalesced along n).
__device__ __forceinline__ int tl_index(int wm, int wn, int i, int j, int lane, int r) {
  return acc_row(wm, i, lane, r) * BN + acc_col(wn, j, lane);
}

#ifdef FDP_PHASE_TIMING
extern __device__ unsigned long long fdp_phase_ts[1024 * 16];
#define FDP_TS(slot)                                                  \
  do {                                                                \
    if (threadIdx.x == 0 && blockIdx.x < 1024)                        \
      fdp_phase_ts[blockIdx.x * 16 + (slot)] = wall_clock64();        \
  } while (0)
#else
#define FDP_TS(slot) \
  do {               \
  } while (0)
#endif


// 16-byte coherent (sc1) stores/loads for the per-group slot exchange.  A slot
// is one 128x128 fp32 tile kept in "thread-major" order: float4 q (0..15) of
// thread t sits at byte (q*256 + t)*16, which makes every wave instruction one
// contiguous 1 KB access.

__device__ inline void slot_store(float* slot, const f32x16 (&v)[2][2]) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(slot, static_cast<short>(0), BM * BN * 4, dma::kRsrcWord3);
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int idx = (a * 2 + c) * 4 + q;
        const f32x4 x = {v[a][c][4 * q], v[a][c][4 * q + 1], v[a][c][4 * q + 2], v[a][c][4 * q + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), r,
                                               (idx * NT + threadIdx.x) * 16, 0, kCoherent);
      }
}
__device__ inline void slot_add(const float* slot, f32x16 (&v)[2][2]) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(slot), static_cast<short>(0), BM * BN * 4, dma::kRsrcWord3);
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int idx = (a * 2 + c) * 4 + q;
        const f32x4 x = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (idx * NT + threadIdx.x) * 16, 0,
                                                         kCoherent));
#pragma unroll
        for (int e = 0; e < 4; ++e) v[a][c][4 * q + e] += x[e];
      }
}

// out[m, n] = out_scale * tot + noise_scale * noise for one 128x128 tile, staged
// through LDS (rows 32q .. 32q+31 in quarter q, 16 KB each, fp32) so that the
// global stores and noise loads are 16-byte row chunks.
__device__ __forceinline__ float* quarter(float* const (&q)[4], int i) {
  switch (i) {
    case 0: return q[0];
    case 1: return q[1];
    case 2: return q[2];
    default: return q[3];
  }
}

template <class OT>
__device__ inline void store_tile_staged(const Args& p, int64_t m0, int64_t n0,
                                         const f32x16 (&tot)[2][2], float* const (&q4)[4]) {
  using S = typename OT::storage;
  constexpr int E = 16 / sizeof(S);  // elements per 16-byte chunk
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    float* qd = quarter(q4, wm / 32 + a);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        qd[(acc_row(0, 0, lane, r)) * BN + acc_col(wn, c, lane)] = tot[a][c][r];
  }
  __syncthreads();
  S* out = static_cast<S*>(p.out);
  const bool vec = (reinterpret_cast<uintptr_t>(out) % 16 == 0) && (p.ldo % E == 0);
  const NoiseSrc nz = p.noise;  // a value copy: no address of the kernel argument is taken
  const int zvec = noise_chunks<E>(nz, p.N);
  constexpr int CPR = BN / E;  // chunks per tile row
#pragma unroll 1
  for (int q = threadIdx.x; q < BM * CPR; q += NT) {
    const int row = q / CPR, col = (q % CPR) * E;
    const int64_t m = m0 + row, n = n0 + col;
    if (m >= p.M || n >= p.N) continue;
    const float* src = quarter(q4, row >> 5) + (row & 31) * BN + col;
    float v[E];
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = src[e] * p.out_scale;
    if (vec && n + E <= p.N) {
      add_noise_chunk<OT, E>(nz, zvec, m * p.N + n, p.noise_scale, v);
      uint4 o;
      S* os = reinterpret_cast<S*>(&o);
#pragma unroll
      for (int e = 0; e < E; ++e) os[e] = OT::from_f32(v[e]);
      *reinterpret_cast<uint4*>(out + m * p.ldo + n) = o;
    } else {
      // right edge or unaligned rows: element stores, noise from whole blocks
      if (nz.z != nullptr) {
      #pragma unroll
        for (int e = 0; e < E; ++e)
          if (n + e < p.N) v[e] += p.noise_scale * nz.at(m * p.N + n + e);
      } else if (nz.draw) {
        float z[E];
        nz.window(m * p.N + n, z);
      #pragma unroll
        for (int e = 0; e < E; ++e) v[e] += p.noise_scale * z[e];
      }
      #pragma unroll
      for (int e = 0; e < E; ++e)
        if (n + e < p.N) out[m * p.ldo + n + e] = OT::from_f32(v[e]);
    }
  }
}

// ------------------------------------------------------ single pass
// Work units of one workgroup: unit j is the 128x128 product of one tile and
// one sample.  The grid is groups x tiles; workgroup (g, tile) holds the tile's
// products of samples chunk_b0 + g*spg + j.  Groups of one tile are combined
// through slots after the grid barrier.
struct UnitMap {
  int tile, nb;
  int64_t b0;
  __device__ __forceinline__ int64_t sample_of(int j) const { return b0 + j; }
};

__device__ inline UnitMap unit_map(const Args& p, int lw, int tiles) {
  UnitMap u{};
  u.tile = lw % tiles;
  const int64_t bend = p.chunk_b0 + p.chunk_nb;
  u.b0 = p.chunk_b0 + int64_t(lw / tiles) * p.spg;
  u.nb = static_cast<int>((u.b0 + p.spg < bend ? u.b0 + p.spg : bend) - u.b0);
  if (u.nb < 0) u.nb = 0;
  return u;
}

// The tile's sum for this launch: added to the running sum of earlier launches
// and kept for later ones (chunk_acc), or written out on the last launch.
__device__ inline void finish_tile(const Args& p, int64_t m0, int64_t n0, f32x16 (&acc)[2][2],
                                   char* st0, char* st1) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  if (!p.chunk_first || !p.chunk_last) {
    // element (a, c, r) sits at row m0 + wm + 32a + 8(r/4) + r%4 + 4(lane/32)
    // and column n0 + wn + 32c + lane%32: a uniform row base plus a 32-bit
    // per-lane offset, so that no 64-bit address is kept per element.
    const int hi = 4 * (lane >> 5);
    const uint32_t loff = static_cast<uint32_t>(hi * p.N + (lane & 31));
    if (m0 + BM <= p.M && n0 + BN <= p.N) {
      // interior tile: straight-line code, every load in flight at once
      if (!p.chunk_first) {
#pragma unroll
        for (int a = 0; a < 2; ++a) {
          float v[2][16];
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float* rp = p.chunk_acc + ((m0 + wm + 32 * a + 8 * (r >> 2) + (r & 3)) * p.N + n0 + wn) + loff;
#pragma unroll
            for (int c = 0; c < 2; ++c) v[c][r] = rp[32 * c];
          }
#pragma unroll
          for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][c][r] += v[c][r];
        }
      }
      if (!p.chunk_last) {
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float* rp = p.chunk_acc + ((m0 + wm + 32 * a + 8 * (r >> 2) + (r & 3)) * p.N + n0 + wn) + loff;
#pragma unroll
            for (int c = 0; c < 2; ++c) rp[32 * c] = acc[a][c][r];
          }
      }
    } else {
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t mrow = m0 + wm + 32 * a + 8 * (r >> 2) + (r & 3);
          if (mrow + hi >= p.M) continue;
          float* rp = p.chunk_acc + (mrow * p.N + n0 + wn);
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            if (n0 + wn + 32 * c + (lane & 31) >= p.N) continue;
            float* e = rp + loff + 32 * c;
            if (!p.chunk_first) acc[a][c][r] += *e;
            if (!p.chunk_last) *e = acc[a][c][r];
          }
        }
    }
  }
  if (p.chunk_last) {
    __syncthreads();  // the staging area may still be read for a previous tile
    float* const q4[4] = {reinterpret_cast<float*>(st0), reinterpret_cast<float*>(st0) + 4096,
                          reinterpret_cast<float*>(st1), reinterpret_cast<float*>(st1) + 4096};
    if (p.out_dtype == FDP_BF16) store_tile_staged<BF16>(p, m0, n0, acc, q4);
    else if (p.out_dtype == FDP_F16) store_tile_staged<F16>(p, m0, n0, acc, q4);
    else store_tile_staged<F32>(p, m0, n0, acc, q4);
    FDP_TS(12);
  }
}

// Workgroups of the grid run their nb products, keeping the finished ones
// packed in AGPRs and the last one live in its accumulators; each product's
// sum of squares goes to partials[sample, tile].  After the grid barrier every
// workgroup knows the norms of its samples and forms sum_b c_b G_b for its
// tile (fixed order: deterministic); the groups of a tile are then combined in
// group order by the last group to arrive, and the result is written (or
// carried to the next launch in chunk_acc).
constexpr int kStages = 2;  // LDS ring depth of the single-pass kernel (64-deep k-tiles)

template <class DT, int U>
__global__ __launch_bounds__(NT, 2) void wgrad_group_kernel(Args p) {
  using G = dma::Geom<BM, BN, 64>;
  static_assert(kStages * G::STAGE == BM * BN * 4, "the output staging reuses the ring");
  __shared__ __attribute__((aligned(16))) char st0[G::STAGE];
  __shared__ __attribute__((aligned(16))) char st1[G::STAGE];
  __shared__ float red[NT / kWave];
  __shared__ float fac[U];
  __shared__ int is_last;
  const dma::Stages stages{{(FDP_LDS char*)(st0), (FDP_LDS char*)(st1),
                            (FDP_LDS char*)(st0), (FDP_LDS char*)(st1)}};
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int tiles = p.tiles_m * p.tiles_n;
  const int lw = logical_wg(blockIdx.x, p.nwg);
  const UnitMap um = unit_map(p, lw, tiles);
  const int nb = um.nb;
  const int nk = static_cast<int>((p.K + G::BK - 1) / G::BK);
  dma::FragOffsets<G> fo;
  fo.init(wm, wn);
  FDP_TS(0);

  // ---- phase 1: the nb products run as one stream of nb*nk k-tiles through
  // the LDS ring, so that the next unit's first k-tiles load while this
  // unit's last ones multiply and its norm is taken.
  const uint16_t* pa = static_cast<const uint16_t*>(p.a);
  const uint16_t* pb = static_cast<const uint16_t*>(p.b);
  Held<true> held[U > 1 ? U - 1 : 1];
  f32x16 acc[2][2];
  zero(acc);
  const int nq = nb * nk;
  dma::Job<G> job;  // loads of k-tile ik of unit iu, the next one to issue
  int iu = 0, ik = 0;
  int64_t m0, n0;
  tile_coords(p, um.tile, m0, n0);
  if (nq > 0) job.init(pa + um.b0 * p.sab, p.lda, pb + um.b0 * p.sbb, p.ldb, p.K, m0, n0);
  auto issue_next = [&](FDP_LDS char* stage) {
    job.issue(stage, ik);
    if (++ik == nk) {
      ik = 0;
      if (++iu < nb) {
        const int64_t b = um.sample_of(iu);
        job.retarget(pa + b * p.sab, p.lda, pb + b * p.sbb, p.ldb, p.K);
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
        dma::compute_stage<DT, G>(stages.get(s), fo, acc);
        if (++ck == nk) {
          // unit cu done.  Rows/columns past M/N may hold the next row's
          // values: leave them out of the norm.
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
          __syncthreads();
          if (threadIdx.x == 0)
            st_coherent(p.partials + um.sample_of(cu) * tiles + um.tile,
                        (red[0] + red[1]) + (red[2] + red[3]));
          FDP_TS(1 + cu);
          if (cu + 1 < nb) {  // park it and start the next product
#pragma unroll
            for (int j = 0; j < U - 1; ++j)
              if (j == cu) held[j].put(acc);
            zero(acc);
          }
          ck = 0;
          ++cu;
        }
      }
    }
  }
  dma::barrier();  // every wave is done reading the ring

  // The tile's hand-over ticket starts at zero in every launch: group 0 clears
  // it before the grid barrier, every ticket is taken after it.  (A ticket
  // word may hold another problem's data: workspace layouts differ by shape.)
  if (threadIdx.x == 0 && p.groups > 1 && lw / tiles == 0)
    __hip_atomic_store(p.tile_turn + um.tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // A wait that expired (only possible when the grid was not resident at once)
  // poisons this workgroup's results with NaN rather than leave them silently
  // wrong; the status word reports it.
  const bool poisoned = grid_barrier(p.bar, unsigned(p.nwg), p.err, p.spin_limit, &is_last);
  FDP_TS(9);

  // ---- clip factors of this workgroup's samples: all partials in one sweep
  float C = p.C, clamp = p.clamp;
  if (p.clip_args_dev != nullptr) {
    C = p.clip_args_dev[0];
    clamp = p.clip_args_dev[1];
  }
  float ps[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    ps[i] = 0.f;
    if (i < nb)
      for (int t = threadIdx.x; t < tiles; t += NT)
        ps[i] += ld_coherent(p.partials + (um.b0 + i) * tiles + t);
  }
  const bool stats_owner = nb > 0 && um.tile == 0;  // one writer per sample
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const float s = wave_sum(ps[i]);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    if (threadIdx.x == 0 && i < nb) {
      const float n = poisoned ? __builtin_nanf("") : sqrtf((red[0] + red[1]) + (red[2] + red[3]));
      const float cf = poisoned ? n : clip_factor(n, C, clamp);
      fac[i] = cf;
      if (stats_owner) {
        if (p.norms_out) p.norms_out[um.b0 + i] = n;
        if (p.factors_out) p.factors_out[um.b0 + i] = cf;
      }
    }
    __syncthreads();
  }
  FDP_TS(14);

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

  // combine the groups of this tile: the last to arrive sums the slots
  const int ngroups = p.groups;
  bool owner = true;
  if (ngroups > 1) {
    const int g = lw / tiles;
    slot_store(p.tile_acc + (int64_t(g) * tiles + um.tile) * (BM * BN), acc);
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
      const unsigned old = __hip_atomic_fetch_add(p.tile_turn + um.tile, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
      is_last = old == unsigned(ngroups - 1);
      // every group has taken its ticket: leave the counter zeroed
      if (is_last)
        __hip_atomic_store(p.tile_turn + um.tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    FDP_TS(10);
    owner = is_last != 0;
    if (owner) {
      zero(acc);
      for (int gg = 0; gg < ngroups; ++gg)
        slot_add(p.tile_acc + (int64_t(gg) * tiles + um.tile) * (BM * BN), acc);
    }
  }
  FDP_TS(11);
  if (owner) finish_tile(p, m0, n0, acc, st0, st1);
  // ---- leave the control words zeroed for the next launch on this
  // workspace: every workgroup has passed the barrier once `done` reaches nwg.
  if (threadIdx.x == 0) {
    const unsigned old =
        __hip_atomic_fetch_add(p.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == unsigned(p.nwg - 1)) {
      __hip_atomic_store(p.bar, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(p.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
constexpr size_t kWsHead = 256;   // err / barrier words at the head of the workspace
constexpr int kGroupUnits = 3;    // samples per group held by one workgroup

// Single-pass geometry for B samples over `tiles` 128x128 tiles on `slots`
// co-resident workgroups: `groups` groups of `spg` samples per launch, units =
// products held by one workgroup (the kernel instance).  groups == 0: more
// tiles than slots, no single pass (the streamed two-pass schedule is used).
struct GroupPlan {
  int groups, spg, units, nwg;
  int64_t chunk;  // samples per launch
};
inline GroupPlan group_plan(int64_t B, int tiles, int slots) {
  GroupPlan g{};
  if (tiles > slots) return g;  // groups == 0
  int64_t G = slots / tiles;
  if (G > B) G = B;
  const int64_t per = (B + G - 1) / G;
  g.spg = static_cast<int>(per < kGroupUnits ? per : kGroupUnits);
  // fewest groups that still cover the chunk with spg samples each
  g.chunk = G * g.spg < B ? G * g.spg : B;
  g.groups = static_cast<int>((g.chunk + g.spg - 1) / g.spg);
  g.units = g.spg;
  g.nwg = g.groups * tiles;
  return g;
}

// `plain`: ordinary dispatch instead of a cooperative launch (the caller
// guarantees that nothing else occupies the device during the call, so the
// grid, sized to the computed occupancy, is resident at once).  `clean`: the
// control words are already zero (every launch of the kernel leaves them so),
// which makes the clearing kernel unnecessary.
template <class DT>
hipError_t try_grouped(Args a, int cus, bool plain, bool clean, hipStream_t s) {
  const int tiles = a.tiles_m * a.tiles_n;
  if (a.K * a.lda * 2 >= (int64_t(1) << 31) || a.K * a.ldb * 2 >= (int64_t(1) << 31))
    return hipErrorNotSupported;
  const GroupPlan gp = group_plan(a.B, tiles, 2 * cus);
  if (gp.groups == 0) return hipErrorNotSupported;
  KernelFn grouped[kGroupUnits] = {&wgrad_group_kernel<DT, 1>, &wgrad_group_kernel<DT, 2>,
                                   &wgrad_group_kernel<DT, 3>};
  KernelFn fn = grouped[gp.units - 1];
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(fn), NT,
                                                   0) != hipSuccess ||
      occ < 2)
    return hipErrorNotSupported;
  a.spg = gp.spg;
  const int64_t words = int64_t(kWsHead / sizeof(unsigned));
  for (int64_t b0 = 0; b0 < a.B; b0 += gp.chunk) {
    Args c = a;
    c.chunk_b0 = b0;
    c.chunk_nb = a.B - b0 < gp.chunk ? a.B - b0 : gp.chunk;
    c.groups = static_cast<int>((c.chunk_nb + gp.spg - 1) / gp.spg);
    c.nwg = c.groups * tiles;
    c.chunk_first = b0 == 0;
    c.chunk_last = b0 + c.chunk_nb >= a.B;
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

// Per-dtype launchers (wgrad_group_{bf16,f16}.hip).
hipError_t launch_grouped_bf16(Args a, int cus, bool plain, bool clean, hipStream_t s);
hipError_t launch_grouped_f16(Args a, int cus, bool plain, bool clean, hipStream_t s);

}  // namespace wg
}  // namespace fdp
