// Clipped per-sample weight-gradient sum on CDNA4 MFMA (gfx950).
//
//   out = out_scale * sum_b c_b * G_b + noise_scale * noise,
//   G_b = a_b^T b_b (TN) or a_b b_b (NN),  c_b = min(clamp, C/(||G_b||_F + 1e-10))
//
// Reference math: flashdp/core/linear_clip.py:94-104 (per-sample einsum, norm,
// clamp, mul, sum) and flashdp/core/bmtm_clip_loop.py:137-173 /
// flashdp/core/bmm_clip_loop.py:129-162 (operator layouts).  The reference
// materialises every G_b in HBM and scales it in a second kernel; here no
// per-sample gradient ever leaves the register file.
//
// Two passes over the operands:
//   pass A (wgrad_norm_kernel): one workgroup per (output tile, sample) runs the
//     tile product on MFMA, squares and sums its fp32 accumulators and writes
//     one partial per (sample, tile) -- a deterministic [B, tiles] buffer.
//   factor (wgrad_factor_kernel): fixed-order sum of each sample's partials ->
//     ||G_b||, c_b.
//   pass B (wgrad_sum_kernel): one workgroup per (output tile, sample group)
//     accumulates the group's samples into ONE fp32 accumulator, rescaling it
//     by c_prev/c_b at each sample boundary so that it always holds
//     sum c_b G_b / c_current; the epilogue multiplies by the last c and applies
//     out_scale and the noise (single group) or writes an fp32 group partial that
//     wgrad_finalize_kernel sums in fixed group order.
//
// Tiles: 128x128 outputs per 256-thread workgroup (4 waves, 64x64 each as 2x2
// blocks of 32x32 MFMA).  16-bit inputs use v_mfma_f32_32x32x16_{bf16,f16} with
// BK=64; fp32 inputs use v_mfma_f32_32x32x2_f32 with BK=16.  Global loads are
// 16-byte and coalesced along the contiguous dimension; for operands whose
// contraction axis is strided (every TN operand) the 16-bit loader transposes
// 4x8 element blocks in registers (v_perm_b32) so that each MFMA lane then reads
// its 8 consecutive k-values with one ds_read_b128.  LDS rows are XOR-swizzled
// in 16-byte chunks to spread both the transposing writes and the fragment
// reads over the banks.  LDS is double-buffered: the next k-tile's global loads
// are issued before the current tile's MFMAs.
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
    char* As[2] = {smem, smem + TILE_BYTES};
    char* Bs[2] = {smem + 2 * TILE_BYTES, smem + 3 * TILE_BYTES};
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int nk = static_cast<int>((p.K + BK - 1) / BK);
    uint4 ra[4], rb[4];
    if (LAYOUT == FDP_LAYOUT_TN) load_kr<VEC>(A, p.lda, p.K, p.M, 0, m0, ra);
    else load_rk<VEC>(A, p.lda, p.K, p.M, 0, m0, ra);
    load_kr<VEC>(Bm, p.ldb, p.K, p.N, 0, n0, rb);
    if (LAYOUT == FDP_LAYOUT_TN) store_kr(As[0], ra);
    else store_rk(As[0], ra);
    store_kr(Bs[0], rb);
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
      mma(As[cur], Bs[cur], acc, wm, wn, lane);
      if (more) {
        if (LAYOUT == FDP_LAYOUT_TN) store_kr(As[cur ^ 1], ra);
        else store_rk(As[cur ^ 1], ra);
        store_kr(Bs[cur ^ 1], rb);
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
    char* As[2] = {smem, smem + TILE_BYTES};
    char* Bs[2] = {smem + 2 * TILE_BYTES, smem + 3 * TILE_BYTES};
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int nk = static_cast<int>((p.K + BK - 1) / BK);
    float4 ra[2], rb[2];
    if (LAYOUT == FDP_LAYOUT_TN) load_kr<VEC>(A, p.lda, p.K, p.M, 0, m0, ra);
    else load_rk<VEC>(A, p.lda, p.K, p.M, 0, m0, ra);
    load_kr<VEC>(Bm, p.ldb, p.K, p.N, 0, n0, rb);
    if (LAYOUT == FDP_LAYOUT_TN) store_kr(As[0], ra);
    else store_rk(As[0], ra);
    store_kr(Bs[0], rb);
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
      mma(As[cur], Bs[cur], acc, wm, wn, lane);
      if (more) {
        if (LAYOUT == FDP_LAYOUT_TN) store_kr(As[cur ^ 1], ra);
        else store_rk(As[cur ^ 1], ra);
        store_kr(Bs[cur ^ 1], rb);
      }
      __syncthreads();
    }
  }
};

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

// ---------------------------------------------------------------- pass A
template <class Core, int LAYOUT, bool VEC>
__global__ __launch_bounds__(NT) void wgrad_norm_kernel(Args p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tile = blockIdx.x;
  const int64_t bidx = blockIdx.y;
  int64_t m0, n0;
  tile_coords(p, tile, m0, n0);
  f32x16 acc[2][2];
  zero(acc);
  Core::template gemm<LAYOUT, VEC>(p, bidx, m0, n0, acc, smem);
  // Out-of-range rows/columns were loaded as zeros, so they add nothing.
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += acc[i][j][r] * acc[i][j][r];
  s = wave_sum(s);
  float* red = reinterpret_cast<float*>(smem);  // gemm() ended on a barrier
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    const int tiles = p.tiles_m * p.tiles_n;
    p.partials[bidx * tiles + tile] = (red[0] + red[1]) + (red[2] + red[3]);
  }
}

// ---------------------------------------------------------------- factors
// One workgroup: ||G_b|| = sqrt(sum over tiles of partials[b, :]) in a fixed
// tree order, c_b = min(clamp, C/(||G_b|| + 1e-10)).
__global__ __launch_bounds__(NT) void wgrad_factor_kernel(const float* partials, int64_t B,
                                                           int tiles, float C, float clamp,
                                                           const float* clip_args_dev,
                                                           int noclip, float* fac_ws,
                                                           float* norms, float* factors) {
  __shared__ float red[NT / kWave];
  if (clip_args_dev != nullptr) {
    C = clip_args_dev[0];
    clamp = clip_args_dev[1];
  }
  for (int64_t b = 0; b < B; ++b) {
    float n = 0.f;
    if (!noclip) {
      float s = 0.f;
      for (int t = threadIdx.x; t < tiles; t += NT) s += partials[b * tiles + t];
      s = wave_sum(s);
      if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
      __syncthreads();
      n = sqrtf((red[0] + red[1]) + (red[2] + red[3]));
      __syncthreads();
    }
    if (threadIdx.x == 0) {
      const float c = noclip ? clamp : clip_factor(n, C, clamp);
      fac_ws[b] = c;
      if (norms) norms[b] = n;
      if (factors) factors[b] = c;
    }
  }
}

// ---------------------------------------------------------------- pass B
template <class Core, int LAYOUT, bool VEC>
__global__ __launch_bounds__(NT) void wgrad_sum_kernel(Args p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tile = blockIdx.x;
  const int g = blockIdx.y;
  int64_t m0, n0;
  tile_coords(p, tile, m0, n0);
  const int64_t b_begin = int64_t(g) * p.spg;
  const int64_t b_end = b_begin + p.spg < p.B ? b_begin + p.spg : p.B;

  f32x16 acc[2][2];
  zero(acc);
  float c_prev = 0.f;
  bool any = false;
  for (int64_t bidx = b_begin; bidx < b_end; ++bidx) {
    const float c = p.factors[bidx];
    if (c == 0.f) continue;  // contributes exactly zero
    if (any) {
      const float ratio = c_prev / c;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] *= ratio;
    }
    Core::template gemm<LAYOUT, VEC>(p, bidx, m0, n0, acc, smem);
    c_prev = c;
    any = true;
  }

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const bool single = p.groups == 1;
  const float scale = any ? c_prev * (single ? p.out_scale : 1.f) : 0.f;
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
        float v = acc[i][j][r] * scale;
        if (single) {
          if (p.noise) v += p.noise_scale * load_as_f32(p.noise, m * p.N + n, p.out_dtype);
          store_from_f32(p.out, m * p.ldo + n, p.out_dtype, v);
        } else {
          p.group_out[(int64_t(g) * p.M + m) * p.N + n] = v;
        }
      }
    }
}

// out = out_scale * sum_g group_out[g] + noise_scale * noise, fixed order in g.
__global__ __launch_bounds__(NT) void wgrad_finalize_kernel(Args p) {
  const int64_t MN = p.M * p.N;
  for (int64_t e = int64_t(blockIdx.x) * NT + threadIdx.x; e < MN; e += int64_t(gridDim.x) * NT) {
    float s = 0.f;
    for (int g = 0; g < p.groups; ++g) s += p.group_out[int64_t(g) * MN + e];
    float v = s * p.out_scale;
    if (p.noise) v += p.noise_scale * load_as_f32(p.noise, e, p.out_dtype);
    const int64_t m = e / p.N, n = e - m * p.N;
    store_from_f32(p.out, m * p.ldo + n, p.out_dtype, v);
  }
}

}  // namespace wg
}  // namespace fdp

// ====================================================================== host
using namespace fdp;
using namespace fdp::wg;

namespace {

constexpr size_t kAlign = 256;
inline size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct Plan {
  int tiles_m, tiles_n, tiles;
  int spg, groups;
  size_t off_partials, off_factors, off_group, total;
};

int num_cus() {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      cus = v;
  }
  return cus;
}

Plan make_plan(int64_t B, int64_t M, int64_t N, int cus) {
  Plan pl{};
  pl.tiles_m = static_cast<int>((M + BM - 1) / BM);
  pl.tiles_n = static_cast<int>((N + BN - 1) / BN);
  pl.tiles = pl.tiles_m * pl.tiles_n;
  // Pass B: split the batch into groups until there are ~2 workgroups per CU,
  // but keep the fp32 group partials (groups*M*N*4 bytes) at or below B*M*N
  // bytes -- well under what one bf16 gradient per sample would occupy.
  int64_t want = (2 * int64_t(cus) + pl.tiles - 1) / pl.tiles;
  const int64_t cap = B / 4 > 1 ? B / 4 : 1;
  if (want > cap) want = cap;
  if (want < 1) want = 1;
  pl.spg = static_cast<int>((B + want - 1) / want);
  pl.groups = static_cast<int>((B + pl.spg - 1) / pl.spg);
  pl.off_partials = 0;
  pl.off_factors = align_up(sizeof(float) * size_t(B) * pl.tiles);
  pl.off_group = pl.off_factors + align_up(sizeof(float) * size_t(B));
  pl.total = pl.off_group + (pl.groups > 1 ? align_up(sizeof(float) * size_t(pl.groups) * M * N) : 0);
  return pl;
}

bool valid_dtype(int d) { return d == FDP_F32 || d == FDP_F16 || d == FDP_BF16; }

template <class Core, int LAYOUT, bool VEC>
hipError_t launch_passes(const Args& a, const Plan& pl, bool noclip, float C, float clamp,
                         const float* clip_args_dev, float* norms, float* factors, float* fac_ws,
                         hipStream_t s) {
  const dim3 block(NT);
  if (!noclip) {
    hipLaunchKernelGGL((wgrad_norm_kernel<Core, LAYOUT, VEC>), dim3(pl.tiles, a.B), block,
                       Core::SMEM, s, a);
  }
  hipLaunchKernelGGL(wgrad_factor_kernel, dim3(1), block, 0, s, a.partials, a.B, pl.tiles, C,
                     clamp, clip_args_dev, noclip ? 1 : 0, fac_ws, norms, factors);
  hipLaunchKernelGGL((wgrad_sum_kernel<Core, LAYOUT, VEC>), dim3(pl.tiles, pl.groups), block,
                     Core::SMEM, s, a);
  if (pl.groups > 1) {
    const int64_t MN = a.M * a.N;
    int64_t nb = (MN + NT - 1) / NT;
    if (nb > 4096) nb = 4096;
    hipLaunchKernelGGL(wgrad_finalize_kernel, dim3(static_cast<unsigned>(nb)), block, 0, s, a);
  }
  return hipGetLastError();
}

template <class Core>
hipError_t dispatch_layout(int layout, bool vec, const Args& a, const Plan& pl, bool noclip,
                           float C, float clamp, const float* cad, float* norms, float* factors,
                           float* fac_ws, hipStream_t s) {
  if (layout == FDP_LAYOUT_TN) {
    return vec ? launch_passes<Core, FDP_LAYOUT_TN, true>(a, pl, noclip, C, clamp, cad, norms,
                                                          factors, fac_ws, s)
               : launch_passes<Core, FDP_LAYOUT_TN, false>(a, pl, noclip, C, clamp, cad, norms,
                                                           factors, fac_ws, s);
  }
  return vec ? launch_passes<Core, FDP_LAYOUT_NN, true>(a, pl, noclip, C, clamp, cad, norms,
                                                        factors, fac_ws, s)
             : launch_passes<Core, FDP_LAYOUT_NN, false>(a, pl, noclip, C, clamp, cad, norms,
                                                         factors, fac_ws, s);
}

}  // namespace

extern "C" int fdp_wgrad_clip_workspace_size(int64_t B, int64_t K, int64_t M, int64_t N,
                                             int dtype, int flags, size_t* bytes) {
  (void)K;
  (void)flags;
  if (bytes == nullptr) return FDP_ERR_ARG;
  if (!valid_dtype(dtype)) return FDP_ERR_DTYPE;
  if (B < 1 || M < 1 || N < 1 || K < 0) return FDP_ERR_SHAPE;
  *bytes = make_plan(B, M, N, num_cus()).total;
  return FDP_OK;
}

extern "C" int fdp_wgrad_clip(const void* a, const void* b, int64_t B, int64_t K, int64_t M,
                              int64_t N, int64_t stride_ab, int64_t lda, int64_t stride_bb,
                              int64_t ldb, int layout, int dtype, float C, float clamp,
                              const float* clip_args_dev, float out_scale, const void* noise,
                              float noise_scale, void* out, int64_t ldo, int out_dtype,
                              float* norms, float* factors, int flags, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) return FDP_ERR_DTYPE;
  if (layout != FDP_LAYOUT_TN && layout != FDP_LAYOUT_NN) return FDP_ERR_ARG;
  if (B < 1 || M < 1 || N < 1 || K < 0) return FDP_ERR_SHAPE;
  if (ldo < N) return FDP_ERR_SHAPE;
  if (layout == FDP_LAYOUT_TN && (lda < M || ldb < N)) return FDP_ERR_SHAPE;
  if (layout == FDP_LAYOUT_NN && (lda < K || ldb < N)) return FDP_ERR_SHAPE;
  if (M * N > (int64_t(1) << 40) || B > (int64_t(1) << 31)) return FDP_ERR_SHAPE;
  if ((K > 0 && (a == nullptr || b == nullptr)) || out == nullptr) return FDP_ERR_ARG;
  if ((flags & ~FDP_WGRAD_NOCLIP) != 0) return FDP_ERR_ARG;
  const bool noclip = (flags & FDP_WGRAD_NOCLIP) != 0;
  if (noclip && norms != nullptr) return FDP_ERR_ARG;

  const Plan pl = make_plan(B, M, N, num_cus());
  if (workspace == nullptr || workspace_bytes < pl.total) return FDP_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) return FDP_ERR_ALIGN;

  char* ws = static_cast<char*>(workspace);
  Args args{};
  args.a = a;
  args.b = b;
  args.B = B;
  args.K = K;
  args.M = M;
  args.N = N;
  args.sab = stride_ab;
  args.lda = lda;
  args.sbb = stride_bb;
  args.ldb = ldb;
  args.tiles_m = pl.tiles_m;
  args.tiles_n = pl.tiles_n;
  args.spg = pl.spg;
  args.groups = pl.groups;
  args.partials = reinterpret_cast<float*>(ws + pl.off_partials);
  float* fac_ws = reinterpret_cast<float*>(ws + pl.off_factors);
  args.factors = fac_ws;
  args.group_out = pl.groups > 1 ? reinterpret_cast<float*>(ws + pl.off_group) : nullptr;
  args.out = out;
  args.ldo = ldo;
  args.out_dtype = out_dtype;
  args.out_scale = out_scale;
  args.noise = noise;
  args.noise_scale = noise_scale;

  // 16-byte vector loads need 16-byte aligned rows of every sample.
  const int esz = dtype == FDP_F32 ? 4 : 2;
  const int64_t vel = 16 / esz;
  const bool vec = (reinterpret_cast<uintptr_t>(a) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(b) % 16 == 0) && lda % vel == 0 &&
                   ldb % vel == 0 && stride_ab % vel == 0 && stride_bb % vel == 0;

  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (dtype == FDP_BF16) {
    e = dispatch_layout<Core16<BF16>>(layout, vec, args, pl, noclip, C, clamp, clip_args_dev,
                                      norms, factors, fac_ws, s);
  } else if (dtype == FDP_F16) {
    e = dispatch_layout<Core16<F16>>(layout, vec, args, pl, noclip, C, clamp, clip_args_dev,
                                     norms, factors, fac_ws, s);
  } else {
    e = dispatch_layout<Core32>(layout, vec, args, pl, noclip, C, clamp, clip_args_dev, norms,
                                factors, fac_ws, s);
  }
  return e == hipSuccess ? FDP_OK : FDP_ERR_HIP;
}
