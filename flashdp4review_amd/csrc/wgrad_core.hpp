// Shared pieces of the clipped per-sample weight-gradient kernels: operand
// loaders and MFMA tile cores for gfx950, and the single-pass cooperative kernel
// template (instantiated per dtype in wgrad_fused_*.hip, launched from
// wgrad_clip.hip).  See wgrad_clip.hip for the algorithm.
#pragma once

#include "fdp_common.hpp"

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
  const void* noise;
  float noise_scale;
  // single-pass (fused) kernel
  int64_t units;          // tiles * B work units, unit u = (tile u/B, sample u%B)
  int nwg;                // workgroups of the cooperative grid
  unsigned* bar;          // grid barrier arrivals
  unsigned* tile_turn;    // [tiles] hand-over tickets for tiles shared by workgroups
  float* tile_acc;        // [tiles, BM*BN] fp32 running sums of shared tiles
  int* err;               // set when a bounded wait gives up
  float C, clamp;
  const float* clip_args_dev;
  float* norms_out;       // optional [B]
  float* factors_out;     // optional [B]
};

// ------------------------------------------------------------------ 16-bit
// LDS tile: [128 rows][64 k] of 16-bit values, 128 bytes per row, in 8 chunks of
// 16 bytes whose position is XOR-swizzled by the row index.
__device__ __forceinline__ int lds16_off(int row, int chunk) {
  return row * 128 + ((chunk ^ ((row ^ (row >> 3)) & 7)) << 4);
}

template <class DT>
struct Core16 {
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

__device__ __forceinline__ void tile_coords(const Args& p, int tile, int64_t& m0, int64_t& n0) {
  m0 = int64_t(tile / p.tiles_n) * BM;
  n0 = int64_t(tile % p.tiles_n) * BN;
}

// ============================================================ single pass
// Persistent cooperative kernel.  The tiles*B units (tile, sample) are split
// into nwg contiguous ranges, sample-minor, so a workgroup's units cover a few
// consecutive tiles for consecutive samples.  Logical workgroup ids are laid out
// so that each of the 8 XCDs runs a contiguous block of ranges (the hardware
// deals workgroups round-robin over the XCDs), which keeps a block's operand
// rows in that XCD's L2.
//
// Phase 1: every unit's 128x128 tile of G_b is computed on MFMA; its sum of
//   squares goes to partials[b, tile] and the tile itself stays in registers
//   (packed to bf16 pairs for 16-bit inputs, fp32 otherwise).
// Grid barrier (all workgroups are co-resident: cooperative launch).
// Phase 2: every workgroup derives all c_b from the partials (same fixed order
//   everywhere), sums c_b * G_b over its units tile by tile and writes tiles it
//   owns entirely.  A tile split between consecutive workgroups is handed from
//   one to the next through tile_acc with a ticket (tile_turn), so its sum is
//   always formed in workgroup order: deterministic, no float atomics.  Each
//   workgroup first finishes the tiles where it is the first contributor and
//   only then waits for its first tile, so hand-over chains are at most as
//   long as the number of workgroups sharing one tile.
// Every wait is bounded (kSpinLimit polls); on expiry err is set and the
// kernel runs to completion, so no wave can be left spinning.
constexpr unsigned kSpinLimit = 1u << 21;
constexpr int kXcds = 8;

__device__ __forceinline__ int64_t unit_begin(int64_t w, int64_t units, int nwg) {
  return w * units / nwg;
}
// The workgroup whose range holds unit u.
__device__ inline int owner_of(int64_t u, int64_t units, int nwg) {
  int w = static_cast<int>((u * nwg) / units);
  while (w > 0 && unit_begin(w, units, nwg) > u) --w;
  while (w + 1 < nwg && unit_begin(w + 1, units, nwg) <= u) ++w;
  return w;
}
__device__ __forceinline__ int logical_wg(int hw, int nwg) {
  if (nwg % kXcds != 0) return hw;
  return (hw % kXcds) * (nwg / kXcds) + hw / kXcds;
}

// Thread 0 polls *p until it reaches `target`; acquire for the whole group.
__device__ inline void wait_at_least(unsigned* p, unsigned target, int* err) {
  if (threadIdx.x == 0) {
    unsigned spins = 0;
    while (__hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < target) {
      __builtin_amdgcn_s_sleep(4);
      if (++spins > kSpinLimit) {
        atomicOr(err, 1);
        break;
      }
    }
  }
  __syncthreads();
  __threadfence();
}

__device__ inline void grid_barrier(unsigned* bar, unsigned nwg, int* err) {
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) atomicAdd(bar, 1u);
  wait_at_least(bar, nwg, err);
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

// out[m, n] = out_scale * tot + noise_scale * noise for the in-range part of a tile.
template <class OT>
__device__ inline void store_tile_t(const Args& p, int64_t m0, int64_t n0,
                                    const f32x16 (&tot)[2][2]) {
  using S = typename OT::storage;
  S* out = static_cast<S*>(p.out);
  const S* noise = static_cast<const S*>(p.noise);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t n = n0 + acc_col(wn, j, lane);
      if (n >= p.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + acc_row(wm, i, lane, r);
        if (m >= p.M) continue;
        float v = tot[i][j][r] * p.out_scale;
        if (noise) v += p.noise_scale * OT::to_f32(noise[m * p.N + n]);
        out[m * p.ldo + n] = OT::from_f32(v);
      }
    }
}
__device__ inline void store_tile(const Args& p, int tile, const f32x16 (&tot)[2][2]) {
  int64_t m0, n0;
  tile_coords(p, tile, m0, n0);
  if (p.out_dtype == FDP_BF16) store_tile_t<BF16>(p, m0, n0, tot);
  else if (p.out_dtype == FDP_F16) store_tile_t<F16>(p, m0, n0, tot);
  else store_tile_t<F32>(p, m0, n0, tot);
}

// Tile-local fp32 buffer access in the accumulator layout (coalesced along n).
__device__ __forceinline__ int tl_index(int wm, int wn, int i, int j, int lane, int r) {
  return acc_row(wm, i, lane, r) * BN + acc_col(wn, j, lane);
}

// Finish one tile of this workgroup's range: write it if owned, otherwise take
// part in the ordered hand-over between the workgroups that share it.
__device__ inline void finish_tile(const Args& p, int lw, int64_t u0, int64_t u1, int tile,
                                   f32x16 (&tot)[2][2]) {
  const int64_t tu0 = int64_t(tile) * p.B, tu1 = tu0 + p.B;
  if (tu0 >= u0 && tu1 <= u1) {
    store_tile(p, tile, tot);
    return;
  }
  const int w0 = owner_of(tu0, p.units, p.nwg);
  const int w1 = owner_of(tu1 - 1, p.units, p.nwg);
  const int k = lw - w0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  float* buf = p.tile_acc + int64_t(tile) * (BM * BN);
  if (k > 0) {
    wait_at_least(p.tile_turn + tile, unsigned(k), p.err);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) tot[i][j][r] = buf[tl_index(wm, wn, i, j, lane, r)] + tot[i][j][r];
  }
  if (lw == w1) {
    store_tile(p, tile, tot);
    return;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) buf[tl_index(wm, wn, i, j, lane, r)] = tot[i][j][r];
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) atomicAdd(p.tile_turn + tile, 1u);
}

template <class Core, int U, bool PACK>
__global__ __launch_bounds__(NT) void wgrad_fused_kernel(Args p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  __shared__ float red[NT / kWave];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lw = logical_wg(blockIdx.x, p.nwg);
  const int64_t u0 = unit_begin(lw, p.units, p.nwg);
  const int64_t u1 = unit_begin(lw + 1, p.units, p.nwg);
  const int nu = static_cast<int>(u1 - u0);
  const int tiles = p.tiles_m * p.tiles_n;

  // ---- phase 1: per-unit tile products, partial norms, tiles kept in registers.
  // One copy of the product loop; the finished tile goes to held[i] through a
  // branch per slot so that every held[] index is a compile-time constant.
  Held<PACK> held[U];
  for (int i = 0; i < nu; ++i) {
    const int64_t u = u0 + i;
    const int tile = static_cast<int>(u / p.B);
    const int64_t bidx = u - int64_t(tile) * p.B;
    int64_t m0, n0;
    tile_coords(p, tile, m0, n0);
    f32x16 acc[2][2];
    zero(acc);
    Core::template gemm<FDP_LAYOUT_TN, true>(p, bidx, m0, n0, acc, smem);
    float s = 0.f;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[a][c][r] * acc[a][c][r];
    s = wave_sum(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    if (threadIdx.x == 0) p.partials[bidx * tiles + tile] = (red[0] + red[1]) + (red[2] + red[3]);
#pragma unroll
    for (int j = 0; j < U; ++j)
      if (j == i) held[j].put(acc);
  }

  grid_barrier(p.bar, unsigned(p.nwg), p.err);

  // ---- clip factors of every sample (identical in every workgroup)
  float C = p.C, clamp = p.clamp;
  if (p.clip_args_dev != nullptr) {
    C = p.clip_args_dev[0];
    clamp = p.clip_args_dev[1];
  }
  float* fac = reinterpret_cast<float*>(smem);
  for (int64_t b = wave; b < p.B; b += NT / kWave) {
    float s = 0.f;
    for (int t = lane; t < tiles; t += kWave) s += p.partials[b * tiles + t];
    const float n = sqrtf(wave_sum(s));
    if (lane == 0) {
      const float c = clip_factor(n, C, clamp);
      fac[b] = c;
      if (lw == 0) {
        if (p.norms_out) p.norms_out[b] = n;
        if (p.factors_out) p.factors_out[b] = c;
      }
    }
  }
  __syncthreads();

  // ---- phase 2: clipped sums per tile.  Tiles whose first unit lies in this
  // range come first (no waiting), the tile begun by an earlier range last.
  const int t_first = static_cast<int>(u0 / p.B);
  const int t_last = nu > 0 ? static_cast<int>((u1 - 1) / p.B) : t_first - 1;
  const bool first_late = (u0 % p.B) != 0 && nu > 0;
  const int t_begin = first_late ? t_first + 1 : t_first;
  const int ntiles = t_last - t_first + 1;
  for (int q = 0; q < ntiles; ++q) {
    const int tile = (t_begin + q <= t_last) ? t_begin + q : t_first;
    f32x16 tot[2][2];
    zero(tot);
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int64_t u = u0 + i;
      if (i < nu && u / p.B == tile) held[i].add_to(tot, fac[u - int64_t(tile) * p.B]);
    }
    finish_tile(p, lw, u0, u1, tile, tot);
  }
}

// Clears the barrier / ticket words at the head of the workspace.
template <int kUnused = 0>
__global__ __launch_bounds__(NT) void clear_words_kernel(unsigned* p, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * NT + threadIdx.x; i < n; i += int64_t(gridDim.x) * NT)
    p[i] = 0u;
}

// ---------------------------------------------------------- single-pass launch
constexpr int kMaxUnits16 = 7;  // 8 would spill (AGPRs full)
constexpr int kMaxUnits32 = 4;
constexpr size_t kWsHead = 256;  // err / barrier words at the head of the workspace

using KernelFn = void (*)(Args);

template <class Core, int U>
KernelFn fused_fn() {
  return &wgrad_fused_kernel<Core, U, (U > 2 && Core::SMEM == Core16<BF16>::SMEM)>;
}

template <class Core>
KernelFn fused_for_units(int u) {
  if constexpr (Core::SMEM == Core32::SMEM) {
    switch (u) {
      case 1: return fused_fn<Core, 1>();
      case 2: return fused_fn<Core, 2>();
      case 3: return fused_fn<Core, 3>();
      case 4: return fused_fn<Core, 4>();
      default: return nullptr;
    }
  } else {
    switch (u) {
      case 1: return fused_fn<Core, 1>();
      case 2: return fused_fn<Core, 2>();
      case 3: return fused_fn<Core, 3>();
      case 4: return fused_fn<Core, 4>();
      case 5: return fused_fn<Core, 5>();
      case 6: return fused_fn<Core, 6>();
      case 7: return fused_fn<Core, 7>();
      case 8: return fused_fn<Core, 8>();
      default: return nullptr;
    }
  }
}

// Tries the single-pass kernel; returns hipErrorNotSupported when the problem
// does not fit it (the caller then runs the two-pass path).
template <class Core>
hipError_t try_fused(Args a, int cus, int max_units, hipStream_t s) {
  const int64_t units = a.units;
  int64_t nwg = units < cus ? units : cus;
  if (nwg >= kXcds) nwg -= nwg % kXcds;
  const int64_t per = (units + nwg - 1) / nwg;
  if (per > max_units) return hipErrorNotSupported;
  KernelFn fn = fused_for_units<Core>(static_cast<int>(per));
  if (fn == nullptr) return hipErrorNotSupported;
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(fn), NT,
                                                   Core::SMEM) != hipSuccess ||
      occ < 1)
    return hipErrorNotSupported;
  a.nwg = static_cast<int>(nwg);
  // Zero the err / barrier words and the tile tickets (one kernel, graph-safe).
  const int64_t words = int64_t(kWsHead / sizeof(unsigned)) + (a.tiles_m * a.tiles_n);
  hipLaunchKernelGGL(clear_words_kernel<0>, dim3(static_cast<unsigned>((words + NT - 1) / NT)),
                     dim3(NT), 0, s, reinterpret_cast<unsigned*>(a.err), words);
  void* params[] = {&a};
  return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(fn), dim3(a.nwg), dim3(NT),
                                    params, Core::SMEM, s);
}


// Per-dtype launchers (wgrad_fused_{bf16,f16,f32}.hip).
hipError_t launch_fused_bf16(Args a, int cus, hipStream_t s);
hipError_t launch_fused_f16(Args a, int cus, hipStream_t s);
hipError_t launch_fused_f32(Args a, int cus, hipStream_t s);

}  // namespace wg
}  // namespace fdp
