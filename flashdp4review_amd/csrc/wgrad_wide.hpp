// Wide single-pass clipped product sum: one (output tile, sample) product per
// CU, held in registers across one grid barrier.
//
//   out = out_scale * sum_b c_b G_b + noise_scale * z,   c_b = clip(||G_b||_F)
//
// Used for 16-bit TN operands when the layer's 384x192 (or 192x384) output
// tiles times the batch fill the device with at most one product per CU --
// e.g. a GPT-2-small MLP weight gradient (768 x 3072 outputs, B = 8: 32 tiles
// x 8 samples = 256 products on 256 CUs).  A workgroup is 8 waves (two per
// SIMD); each wave owns 96 x 96 outputs as 3 x 3 blocks of 32x32 MFMA
// accumulators (144 registers), and the tile streams through a 3-stage ring of
// 32-deep k-tiles (gemm_dma.hpp, gemm_pipe).  Per product:
//
//   1. the product G_b's tile, its masked sum of squares -> partials[b, tile];
//   2. the tile is split into ng regions of whole 32x32 blocks, one per sample
//      of the tile (ng = B, 2 <= B <= 72); the workgroup of sample g
//      stages the blocks of its own region in LDS (bf16) and publishes every
//      other block, unscaled, to its exchange slot (bf16, agent-coherent);
//   3. it arrives at the grid barrier, draws the Gaussian noise of the outputs
//      it will finish while it waits, then leaves;
//   4. it forms the clip factors of the tile's ng samples (each a fixed-order
//      sum of that sample's tile partials) and finishes its region:
//      out = out_scale * sum_g c_g G_g (g in sample order) + noise_scale * z.
//
// No per-sample gradient is written whole: each product leaves the register
// file only as (ng-1)/ng of its tile in bf16 for the exchange.  The result is
// deterministic (fixed summation orders, no float atomics).  Bounded waits
// only: an expired wait sets the status word and this launch's poison tag,
// and the outputs are NaN (the kernel still runs to completion).
#pragma once

#include <type_traits>

#include "wgrad_core.hpp"

namespace fdp {
namespace wg {

constexpr int kWideThreads = 512;   // 8 waves
constexpr int kWideStages = 3;      // LDS ring depth (32-deep k-tiles)
constexpr int kWideBlocks = 72;     // 32x32 blocks per 384x192 tile (8 waves x 3 x 3)
constexpr int kWideBlockBytes = 2 * 64 * 16;  // one 32x32 block in bf16, [half][lane] x 16 bytes
constexpr int kFastGroups = 9;      // samples per tile up to which an item's slots load in one batch
constexpr int kPreNoiseBlocks = 9;  // regions of at most this many blocks (B >= 8) draw their noise early
constexpr int kPreNoiseDraws = 6;   // Philox blocks per thread then: 3 rounds x 2 row groups
constexpr int kPreNoiseEvery = 5;   // k-tiles between two early draws (a draw's VALU work
                                    // exceeds one k-tile's MFMA time)
struct WideArgs {
  const uint16_t* a;
  const uint16_t* b;
  int64_t B, K, M, N;
  int64_t sab, lda, sbb, ldb;
  int tiles_m, tiles_n, tiles;  // the layer's grid of output tiles
  int nwg;                      // workgroups = tiles * B (one product each)
  float* partials;              // [B, tiles] per-product sums of squares
  char* slots;                  // [nwg, slot_blocks * kWideBlockBytes] exchange slots
  int slot_blocks;              // blocks per slot: the tile's blocks outside the smallest region
  void* out;
  int64_t ldo;
  int out_dtype;
  float out_scale;
  NoiseSrc noise;
  float noise_scale;
  unsigned* bar;
  unsigned* epoch;
  unsigned* poison;
  int* err;
  unsigned spin_limit;
  float C, clamp;
  const float* clip_args_dev;
  float* norms_out;
  float* factors_out;
  int vec_out;  // out rows hold whole aligned quads: 4 outputs per vector store
  unsigned* group_cnt;  // paired kernel: [tiles] per-tile counters, then one start
                        // counter (zero between launches)
  uint64_t* tagged;     // paired kernel: [B, tiles] partials, each with its launch tag
  // paired kernel, bias of a (bias_op 1) or b (bias_op 2), tagged like `tagged`:
  uint64_t* bias_tagged;     // [len rounded up to 192][B][P] column sums over a tile's
                             // counted k-tiles (P: tiles along the other axis)
  uint64_t* bias_sq_tagged;  // [B, tiles] their sums of squares
  // The bias of operand a (bias_op 1, rows m) or b (bias_op 2, columns n):
  //   bias[c] = bias_scale * sum_b c'_b sum_k op_b[k, c] + bias_noise_scale * zb[c],
  //   c'_b = clip(||op_b||_F) with the weight's C and clamp.
  int bias_op;       // 0: no bias
  float* bias_part;  // [tiles_own, W, B, tiles_other] (W = the tile's extent along the
                     // bias axis): column sums over a workgroup's k-tiles (an output's
                     // B * tiles_other partials are contiguous)
  float* bias_sq;    // [B, tiles]: sums of squares of the operand over a workgroup's k-tiles
  void* bias_out;
  int bias_dtype;
  float bias_scale;
  NoiseSrc bias_noise;
  float bias_noise_scale;
  float* bias_norms;
  float* bias_factors;
};

// Block bid (0..71) of the tile belongs to region (bid * ng) / 72: ng
// contiguous ranges of whole blocks, one per sample of the tile (ng <= 72).
__device__ __forceinline__ int region_first(int g, int ng) { return (g * kWideBlocks + ng - 1) / ng; }
// Position of block bid in the slot of the sample whose region is [r0, r1)
// (a slot holds every block outside its own region, in block order).
__device__ __forceinline__ int slot_block(int bid, int r0, int r1) { return bid < r0 ? bid : bid - (r1 - r0); }

// 4x4 transpose inside each quad of lanes: lane k of the quad holds in[0..3]
// (row k, columns 0..3 of the quad's 4 columns); it returns column k, rows 0..3.
__device__ __forceinline__ void quad_transpose(const float (&in)[4], float (&out)[4]) {
  const int k = threadIdx.x & 3;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    // lane r provides in[(r - s) & 3]; lane k receives it from lane (k + s) & 3
    const int e = (k - s) & 3;
    const float v = e == 0 ? in[0] : e == 1 ? in[1] : e == 2 ? in[2] : in[3];
    // quad_perm controls with lane k reading lane (k + s) & 3: 0x39, 0x4E, 0x93
    const float r =
        s == 0 ? v
        : s == 1 ? __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x39, 0xf, 0xf, false))
        : s == 2 ? __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xf, 0xf, false))
                 : __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x93, 0xf, 0xf, false));
    const int d = (k + s) & 3;
    out[0] = d == 0 ? r : out[0];
    out[1] = d == 1 ? r : out[1];
    out[2] = d == 2 ? r : out[2];
    out[3] = d == 3 ? r : out[3];
  }
}

// Stores one finish item: the 8 sums v of rows mr + {0..3, 8..11} of column
// nc (registers 8h..8h+7 of one lane of a 32x32 block), as
// out = out_scale * v + noise_scale * z.  Each 4-row group is transposed in
// its quad of lanes: lane k then holds row k's 4 consecutive outputs, one
// vector store (and the row layout of the Philox draw).  zpre: the item's two
// early draws (row groups 0 and 1), or nullptr to draw them here.
__device__ __forceinline__ void store_item(const WideArgs& p, const NoiseSrc& nz, const f32x4* zpre,
                                           int64_t mr, int64_t nc, const float (&v)[8],
                                           bool poisoned) {
  const int lane = threadIdx.x & 63;
  const int64_t n4 = nc & ~int64_t(3);
#pragma unroll 1
  for (int grp = 0; grp < 2; ++grp) {
    float src[4], o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) src[k] = (grp == 0 ? v[k] : v[4 + k]) * p.out_scale;
    quad_transpose(src, o);
    const int64_t row = mr + 8 * grp + (lane & 3);
    if (nz.on()) {
      float z[4];
      if (zpre != nullptr) {
        const f32x4 zz = zpre[grp];
#pragma unroll
        for (int c = 0; c < 4; ++c) z[c] = zz[c];
      } else if (nz.z == nullptr && p.N % 4 == 0) {
        nz.block((row * p.N + n4) / 4, z);
      } else {
        // an injected tensor, or rows of N % 4 != 0 outputs: element by
        // element (rolled: one copy of the element draw, placed by selects)
#pragma unroll
        for (int c = 0; c < 4; ++c) z[c] = 0.f;
#pragma unroll 1
        for (int c = 0; c < 4; ++c) {
          const float zc = (row < p.M && n4 + c < p.N) ? nz.at(row * p.N + n4 + c) : 0.f;
#pragma unroll
          for (int q = 0; q < 4; ++q) z[q] = q == c ? zc : z[q];
        }
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] += p.noise_scale * z[c];
    }
    if (poisoned) {
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = __builtin_nanf("");
    }
    if (row < p.M) {
      const int64_t e = row * p.ldo + n4;
      if (p.out_dtype == FDP_F32) {
        float* out = static_cast<float*>(p.out) + e;
        if (p.vec_out && n4 + 4 <= p.N) {
          *reinterpret_cast<f32x4*>(out) = f32x4{o[0], o[1], o[2], o[3]};
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (n4 + c < p.N) out[c] = o[c];
        }
      } else {
        uint16_t h16[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
          h16[c] = p.out_dtype == FDP_BF16 ? BF16::from_f32(o[c]) : F16::from_f32(o[c]);
        uint16_t* out = static_cast<uint16_t*>(p.out) + e;
        if (p.vec_out && n4 + 4 <= p.N) {
          *reinterpret_cast<uint2*>(out) =
              make_uint2(uint32_t(h16[0]) | (uint32_t(h16[1]) << 16),
                         uint32_t(h16[2]) | (uint32_t(h16[3]) << 16));
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (n4 + c < p.N) out[c] = h16[c];
        }
      }
    }
  }
}

// BOP 1 / 2: also the bias of operand a / b, from the fragments the MFMAs
// already hold (bias_frag): k-tile kt is counted by the tile whose index along
// the other axis is kt % (tiles there), k-step ks by the wave with index ks
// among the waves that share the fragment; the workgroup folds its waves'
// column sums through LDS and publishes them, and after the barrier workgroup
// L finishes bias outputs [L * ceil(len / nwg), ...).
template <class DT, int WGM, int WGN, int BOP>
__global__ __launch_bounds__(kWideThreads, 1) void wgrad_wide_kernel(WideArgs p) {
  constexpr bool BIAS = BOP != 0;
  using G = dma::Geom<96 * WGM, 96 * WGN, 32, WGM, WGN>;
  static_assert(G::NW == 8 && G::FI == 3 && G::FJ == 3, "8 waves of 3x3 blocks");
  constexpr int S = kWideStages;
  __shared__ __attribute__((aligned(16))) char st0[G::STAGE];
  __shared__ __attribute__((aligned(16))) char st1[G::STAGE];
  __shared__ __attribute__((aligned(16))) char st2[G::STAGE];
  __shared__ float red[8];
  __shared__ float fac[kWideBlocks];  // clip factors of the tile's samples (ng <= 72)
  __shared__ float bfac[BIAS ? kWideBlocks : 1];  // bias clip factors
  __shared__ int flag;
  // The own region (at most 36 blocks when ng >= 2) is staged in the free ring,
  // kStageBlocks whole blocks per stage array.
  constexpr int kStageBlocks = G::STAGE / kWideBlockBytes;
  static_assert(3 * kStageBlocks >= kWideBlocks / 2, "own region staging fits the ring");
  const dma::Stages stages{{(FDP_LDS char*)(st0), (FDP_LDS char*)(st1), (FDP_LDS char*)(st2),
                            (FDP_LDS char*)(st0)}};
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave / WGN) * 96, wn = (wave % WGN) * 96;

  // hardware workgroup -> (sample, tile), sample-major.  Workgroups are dealt
  // round-robin to the 8 XCDs (the starting XCD varies from launch to launch,
  // but workgroups hw and hw + 8 always share one), and logical_wg gives each
  // such set a contiguous range of units: the workgroups of one XCD read the
  // same sample's operands through its L2.  The placement only affects speed.
  const int hw = blockIdx.x;
  const int L = logical_wg(hw, p.nwg);
  const int ng = static_cast<int>(p.B);
  const int sample = L / p.tiles, tile = L % p.tiles;
  int64_t m0, n0;
  {
    // bands of kBandRows tile rows walked column by column
    const int per_band = kBandRows * p.tiles_n;
    const int band = tile / per_band, in_band = tile % per_band;
    const int rows_left = p.tiles_m - band * kBandRows;
    const int band_rows = rows_left < kBandRows ? rows_left : kBandRows;
    m0 = int64_t(band * kBandRows + in_band % band_rows) * G::BM;
    n0 = int64_t(in_band / band_rows) * G::BN;
  }
  unsigned tag = 0;
  if (threadIdx.x == 0)
    tag = __hip_atomic_load(p.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;

  // the region of the tile this workgroup finishes (step 2), and its items:
  // item it = (block rb0 + it/128, half (it/64)%2, lane it%64), the 8 outputs
  // of registers 8h..8h+7 of that lane: rows mrow + {0..3, 8..11}, column ncol
  const int g = sample;
  const int rb0 = region_first(g, ng), rb1 = region_first(g + 1, ng);
  const int nitems = (rb1 - rb0) * 128;
  auto item_pos = [&](int it, int64_t& mrow, int64_t& ncol) {
    const int bid = rb0 + it / 128, h = (it >> 6) & 1;
    const int w = bid / 9, ij = bid % 9;
    const int i = ij / 3, j = ij % 3;
    const int l = it & 63;
    mrow = m0 + (w / WGN) * 96 + 32 * i + 16 * h + 4 * (l >> 5);
    ncol = n0 + (w % WGN) * 96 + 32 * j + (l & 31);
  };
  // Noise.  Lane k of each quad of lanes (4 adjacent columns) draws the Philox
  // block of row k of each 4-row group: four normals of 4 consecutive outputs
  // of one row, the layout the finish stores in.  With B >= 8 (regions of at
  // most 9 blocks) and whole blocks per row (N % 4 == 0, no injected tensor)
  // the draws happen during the product phase, one per k-tile while the
  // matrix cores work, into LDS; otherwise in the finish.
  const NoiseSrc nz = p.noise.resolved();
  const bool noisy = nz.on();
  const bool pre_noise = noisy && nz.z == nullptr && p.N % 4 == 0 && rb1 - rb0 <= kPreNoiseBlocks;
  __shared__ f32x4 zpre[kPreNoiseBlocks * 128 * 2];
  auto draw_early = [&](int j) {  // draw j: round j/2, row group j%2
    const int it = threadIdx.x + (j >> 1) * kWideThreads;
    if (it < nitems) {
      int64_t mr, nc;
      item_pos(it, mr, nc);
      const int64_t row = mr + 8 * (j & 1) + (lane & 3);
      float blk[4];
      nz.block((row * p.N + (nc & ~int64_t(3))) / 4, blk);
      zpre[it * 2 + (j & 1)] = f32x4{blk[0], blk[1], blk[2], blk[3]};
    }
  };

  // bias: this lane's columns of the bias operand (wm + 32 i + lane % 32 of a,
  // or wn + 32 j + lane % 32 of b; k half lane / 32)
  const int tile_m = static_cast<int>(m0 / G::BM), tile_n = static_cast<int>(n0 / G::BN);
  const int blim = bias_limit(BOP == 1 ? p.M : p.N, BOP == 1 ? m0 : n0);
  float bcs[3] = {0.f, 0.f, 0.f}, bsq = 0.f;
  auto fhook = [&](int kt, int ks, const dma::Frags<G>& f) {
    if constexpr (BOP == 1) {
      if (kt % p.tiles_n == tile_n && (wave % WGN) == ks) {
#pragma unroll
        for (int i = 0; i < 3; ++i)
          bias_frag<DT>(f.a[i], bcs[i], bsq, wm + 32 * i + (lane & 31), blim);
      }
    } else if constexpr (BOP == 2) {
      if (kt % p.tiles_m == tile_m && (wave / WGN) == ks) {
#pragma unroll
        for (int j = 0; j < 3; ++j)
          bias_frag<DT>(f.b[j], bcs[j], bsq, wn + 32 * j + (lane & 31), blim);
      }
    }
  };

  // ---- 1. the product
  f32x16 acc[3][3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  {
    dma::FragOffsets<G> fo;
    fo.init(wm, wn);
    dma::Job<G> job;
    job.init(p.a + sample * p.sab, p.lda, p.b + sample * p.sbb, p.ldb, p.K, m0, n0);
    const int nk = static_cast<int>((p.K + G::BK - 1) / G::BK);
    // draw j at k-tile (j + 1) * kPreNoiseEvery; draws the contraction is too
    // short for follow the product phase
    auto hook = [&](int kt) {
      if (pre_noise && kt > 0 && kt % kPreNoiseEvery == 0 && kt / kPreNoiseEvery <= kPreNoiseDraws)
        draw_early(kt / kPreNoiseEvery - 1);
    };
    dma::gemm_pipe<DT, G, S>(job, nk, fo, stages, acc, hook, fhook);
    if (pre_noise) {
      const int done = (nk - 1) / kPreNoiseEvery;  // draws made inside the loop
#pragma unroll 1
      for (int j = done < kPreNoiseDraws ? done : kPreNoiseDraws; j < kPreNoiseDraws; ++j)
        draw_early(j);
    }
  }
  if constexpr (BIAS) {
    // lanes l and l + 32 hold one column's two k halves; the NS waves sharing
    // a fragment (one k-step each) are added in wave order through LDS (st2 is
    // free: gemm_pipe ended on a barrier, and the own region never reaches it)
    constexpr int W = BOP == 1 ? G::BM : G::BN;  // the tile's extent along the bias axis
    constexpr int NS = BOP == 1 ? WGN : WGM;     // waves sharing a fragment
    __shared__ float bred[8];
    float* colp = reinterpret_cast<float*>(st2);  // [NS][W]
    const int ws = BOP == 1 ? wave % WGN : wave / WGN;
    const int cl0 = BOP == 1 ? wm : wn;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const float v = bcs[i] + __shfl_xor(bcs[i], 32, kWave);
      if (lane < 32) colp[ws * W + cl0 + 32 * i + lane] = v;
    }
    const float q = wave_sum_dpp(bsq);
    if (lane == 0) bred[wave] = q;
    __syncthreads();
    const int tiles_o = BOP == 1 ? p.tiles_n : p.tiles_m;
    const int own = BOP == 1 ? tile_m : tile_n, oth = BOP == 1 ? tile_n : tile_m;
    const int J = ng * tiles_o;  // partials per output
    float* part = p.bias_part + int64_t(own) * W * J + sample * tiles_o + oth;
    for (int r = threadIdx.x; r < W; r += kWideThreads) {
      float v = colp[r];
#pragma unroll
      for (int q2 = 1; q2 < NS; ++q2) v += colp[q2 * W + r];
      st_coherent(part + int64_t(r) * J, v);
    }
    if (threadIdx.x == 0)
      st_coherent(p.bias_sq + int64_t(sample) * p.tiles + tile,
                  ((bred[0] + bred[1]) + (bred[2] + bred[3])) + ((bred[4] + bred[5]) + (bred[6] + bred[7])));
  }
  {
    // rows/columns past M/N may hold the next row's values: left out of the norm
    // (32-bit tile-local bounds; a tile inside the matrix skips the masks)
    const int64_t rl = p.M - m0, cl = p.N - n0;
    const int rlim = rl < G::BM ? static_cast<int>(rl) : G::BM;
    const int clim = cl < G::BN ? static_cast<int>(cl) : G::BN;
    float sq = 0.f;
    if (rlim == G::BM && clim == G::BN) {
#pragma unroll
      for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) sq = __builtin_fmaf(acc[i][j][r], acc[i][j][r], sq);
    } else {
#pragma unroll
      for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const bool ncol = acc_col(wn, j, lane) < clim;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float v = ncol && acc_row(wm, i, lane, r) < rlim ? acc[i][j][r] : 0.f;
            sq = __builtin_fmaf(v, v, sq);
          }
        }
    }
    sq = wave_sum_dpp(sq);
    if (lane == 0) red[wave] = sq;
    __syncthreads();
    if (threadIdx.x == 0)
      st_coherent(p.partials + int64_t(sample) * p.tiles + tile,
                  ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7])));
  }

  // ---- 2. own region to LDS, the other blocks to the exchange slot (bf16)
  const int slot_bytes = p.slot_blocks * kWideBlockBytes;
  // own-region block lb, half h, lane l: 16 bytes in the ring (free: gemm_pipe
  // ended on a barrier)
  auto own_at = [&](int lb, int h, int l) -> char* {
    char* base = lb < kStageBlocks ? st0 : lb < 2 * kStageBlocks ? st1 : st2;
    return base + ((lb % kStageBlocks) * 2 + h) * 1024 + l * 16;
  };
  {
    const CoherentSpan slot(reinterpret_cast<const float*>(p.slots + int64_t(L) * slot_bytes),
                            static_cast<uint32_t>(slot_bytes));
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const int bid = wave * 9 + i * 3 + j;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          u32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            w[e] = BF16::pack2(acc[i][j][8 * h + 2 * e], acc[i][j][8 * h + 2 * e + 1]);
          if (bid < rb0 || bid >= rb1) {
            slot.store4(static_cast<uint32_t>((slot_block(bid, rb0, rb1) * 2 + h) * 1024 + lane * 16),
                        __builtin_bit_cast(f32x4, w));
          } else {
            *reinterpret_cast<u32x4*>(own_at(bid - rb0, h, lane)) = w;
          }
        }
      }
  }

  // ---- 3. the grid barrier (every workgroup carries the same work, so the
  // waits are short: poll with short sleeps)
  const unsigned arrival = grid_arrive(p.bar);
  bool poisoned = grid_wait(p.bar, unsigned(p.nwg), arrival, p.err, p.epoch, p.poison, tag,
                            p.spin_limit, &flag, 0, 2);

  // ---- 4. clip factors of the tile's samples (wave w: samples w, w + 8, ...)
  {
    float C = p.C, clamp = p.clamp;
    if (p.clip_args_dev != nullptr) {
      C = p.clip_args_dev[0];
      clamp = p.clip_args_dev[1];
    }
    for (int s = wave; s < ng; s += 8) {
      const float* part = p.partials + int64_t(s) * p.tiles;
      float acc_s = 0.f;
      for (int t = lane; t < p.tiles; t += kWave) acc_s += ld_coherent(part + t);
      acc_s = wave_sum_dpp(acc_s);
      if (lane == 0) {
        const float n = poisoned ? __builtin_nanf("") : sqrtf(acc_s);
        const float cf = poisoned ? n : clip_factor(n, C, clamp);
        fac[s] = cf;
        if (tile == 0 && s == sample) {  // one writer per sample
          if (p.norms_out) p.norms_out[s] = n;
          if (p.factors_out) p.factors_out[s] = cf;
        }
      }
      if constexpr (BIAS) {
        const float* bpart = p.bias_sq + int64_t(s) * p.tiles;
        float bq = 0.f;
        for (int t = lane; t < p.tiles; t += kWave) bq += ld_coherent(bpart + t);
        bq = wave_sum_dpp(bq);
        if (lane == 0) {
          const float n = poisoned ? __builtin_nanf("") : sqrtf(bq);
          const float cf = poisoned ? n : clip_factor(n, C, clamp);
          bfac[s] = cf;
          if (tile == 0 && s == sample) {
            if (p.bias_norms) p.bias_norms[s] = n;
            if (p.bias_factors) p.bias_factors[s] = cf;
          }
        }
      }
    }
    __syncthreads();  // (also: the own region is staged)
  }

  // ---- 4b. the bias: workgroup L finishes outputs [L * per, (L + 1) * per),
  // one per thread: sum over (sample s, k-range q) in that order of
  // c'_s * part[s][q]; an output's partials are contiguous, loaded as 16-byte
  // agent-coherent vectors, 8 in flight at a time
  if constexpr (BIAS) {
    constexpr int W = BOP == 1 ? G::BM : G::BN;
    const int64_t len = BOP == 1 ? p.M : p.N;
    const int tiles_o = BOP == 1 ? p.tiles_n : p.tiles_m;
    const int64_t per = (len + p.nwg - 1) / p.nwg;
    const int J = ng * tiles_o;
    const uint32_t pbytes =
        static_cast<uint32_t>(int64_t(BOP == 1 ? p.tiles_m : p.tiles_n) * W * J * 4);
    const CoherentSpan span(p.bias_part, pbytes);
    for (int64_t m = int64_t(L) * per + threadIdx.x;
         m < len && m < (int64_t(L) + 1) * per; m += kWideThreads) {
      const uint32_t base = static_cast<uint32_t>(m * J * 4);
      float v = 0.f;
      if (J % 4 == 0) {
#pragma unroll 1
        for (int j0 = 0; j0 < J; j0 += 32) {
          f32x4 x[8];
#pragma unroll
          for (int u = 0; u < 8; ++u)
            x[u] = j0 + 4 * u < J ? span.load4(base + (j0 + 4 * u) * 4) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int u = 0; u < 8; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (j0 + 4 * u + e < J) v += bfac[(j0 + 4 * u + e) / tiles_o] * x[u][e];
        }
      } else {
#pragma unroll 1
        for (int j = 0; j < J; ++j) v += bfac[j / tiles_o] * ld_coherent(p.bias_part + m * J + j);
      }
      v *= p.bias_scale;
      if (p.bias_noise.on()) v += p.bias_noise_scale * p.bias_noise.at(m);
      if (poisoned) v = __builtin_nanf("");
      store_from_f32(p.bias_out, m, p.bias_dtype, v);
    }
  }

  // ---- 5. finish: out = out_scale * sum_g c_g G_g + noise_scale * z, one item
  // per thread and round.  Rolled loops: the code of a round must stay small
  // enough for the instruction cache.
  const int l = lane;
  const int64_t slot_stride = int64_t(p.tiles) * slot_bytes;  // between samples of one tile
  const char* const slots_tile = p.slots + int64_t(tile) * slot_bytes;
  // exchange chunk of sample gg for block bid, half h (this thread's lane)
  auto slot_load = [&](int gg, int bid, int h) -> u32x4 {
    const CoherentSpan sl(reinterpret_cast<const float*>(slots_tile + gg * slot_stride),
                          static_cast<uint32_t>(slot_bytes));
    const int sb = slot_block(bid, region_first(gg, ng), region_first(gg + 1, ng));
    return __builtin_bit_cast(u32x4, sl.load4(static_cast<uint32_t>((sb * 2 + h) * 1024 + l * 16)));
  };
  auto chunk = [&](int gg, int bid, int h) -> u32x4 {
    return gg == g ? *reinterpret_cast<const u32x4*>(own_at(bid - rb0, h, l)) : slot_load(gg, bid, h);
  };
  auto add_scaled = [&](float (&v)[8], const u32x4& w, float c) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] += c * __uint_as_float(w[e] << 16);
      v[2 * e + 1] += c * __uint_as_float(w[e] & 0xffff0000u);
    }
  };
  auto finish = [&](int it, const float (&v)[8]) {
    int64_t mr, nc;
    item_pos(it, mr, nc);
    store_item(p, nz, pre_noise ? zpre + it * 2 : nullptr, mr, nc, v, poisoned);
  };
  if (ng >= 8 && ng <= kFastGroups) {
    // at most 3 items per thread (regions of 8 or 9 blocks): every chunk of
    // every item is loaded first (up to 27 loads in flight), then summed
    constexpr int R = 3;
    static_assert((kWideBlocks / 8 + 1) * 128 <= R * kWideThreads, "3 rounds cover a region");
    u32x4 w[R][kFastGroups];
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int it = threadIdx.x + k * kWideThreads;
      if (it < nitems) {
        const int bid = rb0 + it / 128, h = (it >> 6) & 1;
#pragma unroll
        for (int gg = 0; gg < kFastGroups; ++gg)
          if (gg < ng) w[k][gg] = chunk(gg, bid, h);
      }
    }
#pragma unroll 1
    for (int k = 0; k < R; ++k) {
      const int it = threadIdx.x + k * kWideThreads;
      if (it >= nitems) break;
      float v[8] = {};
      // (round k's chunks through selects: the register arrays stay static)
#pragma unroll
      for (int gg = 0; gg < kFastGroups; ++gg)
        if (gg < ng) add_scaled(v, k == 0 ? w[0][gg] : k == 1 ? w[1][gg] : w[2][gg], fac[gg]);
      finish(it, v);
    }
  } else if (ng <= kFastGroups) {
    // all chunks of an item in one batch; the next item's batch is issued
    // before this one is summed
    u32x4 cur[kFastGroups], nxt[kFastGroups];
    auto issue = [&](int it, u32x4 (&dst)[kFastGroups]) {
      const int bid = rb0 + it / 128, h = (it >> 6) & 1;
#pragma unroll
      for (int gg = 0; gg < kFastGroups; ++gg)
        if (gg < ng) dst[gg] = chunk(gg, bid, h);
    };
    if (threadIdx.x < nitems) issue(threadIdx.x, cur);
#pragma unroll 1
    for (int it = threadIdx.x; it < nitems; it += kWideThreads) {
      if (it + kWideThreads < nitems) issue(it + kWideThreads, nxt);
      float v[8] = {};
#pragma unroll
      for (int gg = 0; gg < kFastGroups; ++gg)
        if (gg < ng) add_scaled(v, cur[gg], fac[gg]);
      finish(it, v);
#pragma unroll
      for (int gg = 0; gg < kFastGroups; ++gg) cur[gg] = nxt[gg];
    }
  } else {
#pragma unroll 1
    for (int it = threadIdx.x; it < nitems; it += kWideThreads) {
      const int bid = rb0 + it / 128, h = (it >> 6) & 1;
      float v[8] = {};
      // chunks in sample order, 8 loads in flight at a time
#pragma unroll 1
      for (int gb = 0; gb < ng; gb += 8) {
        u32x4 wb[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          wb[u] = gb + u < ng ? chunk(gb + u, bid, h) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (gb + u < ng) add_scaled(v, wb[u], fac[gb + u]);
      }
      finish(it, v);
    }
  }
}

// ================================================================ paired
// Two samples' products of one 192x192 output tile per CU, added inside the
// CU.  For the wide schedule's shapes with an even batch (6 <= B <= 72) and
// whole 32-deep k-tiles: a GPT-2-small MLP weight gradient at B = 8 is
// 64 tiles x 4 sample pairs = 256 workgroups on 256 CUs.  Waves 0-3 hold the
// first sample's 2 x 2 wave tiles of 96 x 96 (3 x 3 blocks of 32x32 MFMA
// accumulators, as in the wide kernel), waves 4-7 the second sample's; one
// LDS stage holds both samples' k-tiles side by side (rows of 384 values, no
// padding), 3 stages in 144 KB.  Per workgroup:
//
//   1. the two products, their masked sums of squares -> partials[b, tile],
//      each stored with the launch's tag in one 64-bit word;
//   2. two waves poll the pair's partials (all tiles of its two samples)
//      until every one carries the tag, and form the two clip factors c;
//   3. S = c_2q G_2q + c_2q+1 G_2q+1 in fp32 (for each block one of the two
//      waves holding it hands its scaled block to the other through LDS);
//   4. the tile's 36 blocks are split into ng = B/2 regions, one per pair; the
//      workgroup keeps its own region of S in LDS (fp32) and publishes every
//      other block (bf16, agent-coherent) to its exchange slot, then draws
//      the noise of its region (into LDS) while those stores drain;
//   5. the ng workgroups of the tile wait for each other;
//   6. finish: out = out_scale * sum_q S_q (q in pair order) + noise.
//
// The tile's wait uses a self-resetting counter per tile (grid_wait) at the
// head of the workspace.  No grid-wide barrier: a pair's clip factors depend
// on its own workgroups only.
//
// Against the wide kernel's one product per CU this loads a third more
// operand bytes per flop (each k-tile carries 4 x 192 columns for 2 x 192^2
// outputs instead of 576 for 384 x 192), and exchanges (ng-1)/ng of one
// clipped pair sum per CU instead of of every product: 14 MB instead of
// 33 MB at B = 8.  Sums are formed in fixed orders: deterministic.
struct PairGeom {
  static constexpr int BM = 384, BN = 384;  // LDS rows: both samples' 192 columns
  static constexpr int BK = 32;
  static constexpr int NW = 8, KS = BK / 16;
  static constexpr int WM = 96, WN = 96, FI = 3, FJ = 3;
  static constexpr bool AKC = false, BKC = false;  // both operands k-strided
  static constexpr int ROW_A = dma::row_chunks(BM) * 16;
  static constexpr int ROW_B = dma::row_chunks(BN) * 16;
  static constexpr int TILE_A = BK * ROW_A;
  static constexpr int TILE_B = BK * ROW_B;
  static constexpr int STAGE = TILE_A + TILE_B;
  static constexpr int LOADS_A = TILE_A / (NW * 64 * 16);
  static constexpr int LOADS_B = TILE_B / (NW * 64 * 16);
  static constexpr int LOADS = LOADS_A + LOADS_B;
  static_assert(LOADS_A * NW * 64 * 16 == TILE_A && LOADS_B * NW * 64 * 16 == TILE_B,
                "each wave issues whole 1 KB loads");
};
constexpr int kPairTile = 192;
constexpr int kPairBlocks = 36;      // 32x32 blocks per 192x192 tile
constexpr int kPairMinB = 6;         // regions of at most 12 blocks (48 KB in fp32)
constexpr int kPairRegionMax = 12;
constexpr int kPairFast = 8;         // pairs up to which a round's chunks load at once

__device__ __forceinline__ int pair_region_first(int q, int ng) {
  return (q * kPairBlocks + ng - 1) / ng;
}

// BOP 1 / 2: also the bias of operand a / b (the counting rule of the wide
// kernel: k-tile kt is counted by the tile whose index along the other axis is
// kt % (tiles there), k-step ks by the sample's wave with index ks among the
// two that share the fragment).  Each workgroup publishes its two samples'
// column sums and squares as tagged words right after the products, and
// finishes bias outputs [L * ceil(len / nwg), ...) at the end, when they have
// long been visible.
template <class DT, int BOP>
__global__ __launch_bounds__(kWideThreads, 1) void wgrad_pair_kernel(WideArgs p) {
  constexpr bool BIAS = BOP != 0;
  using G = PairGeom;
  constexpr int S = kWideStages;
  __shared__ __attribute__((aligned(16))) char st0[G::STAGE];
  __shared__ __attribute__((aligned(16))) char st1[G::STAGE];
  __shared__ __attribute__((aligned(16))) char st2[G::STAGE];
  __shared__ float red[8];
  __shared__ float fac[2];
  __shared__ int bad2[2];
  __shared__ float bred[8];
  __shared__ float bfac[BIAS ? kWideBlocks : 1];  // bias clip factors (B <= 72)
  __shared__ int bbad;
  __shared__ unsigned tag_s;
  __shared__ int flag;
  static_assert(4 * 3 * 16 * 64 * 4 <= G::STAGE, "a row of scaled blocks fits a stage");
  static_assert(kPairRegionMax * 16 * 64 * 4 <= G::STAGE, "the own region fits a stage");
  static_assert(kPairRegionMax * 128 * 2 * 16 <= G::STAGE, "the region's noise fits a stage");
  static_assert(kPairRegionMax * 1024 * 4 <= G::STAGE, "the region's sums fit a stage");
  const dma::Stages stages{{(FDP_LDS char*)(st0), (FDP_LDS char*)(st1), (FDP_LDS char*)(st2),
                            (FDP_LDS char*)(st0)}};
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = wave >> 2, wl = wave & 3;  // sample of the pair, wave within the sample
  const int wm = (wl >> 1) * 96, wn = (wl & 1) * 96;

  // hardware workgroup -> (pair, tile), pair-major: the workgroups of one XCD
  // (logical_wg) contract one pair's operands over a band of tiles
  const int L = logical_wg(blockIdx.x, p.nwg);
  const int ng = static_cast<int>(p.B / 2);
  const int q = L / p.tiles, tile = L % p.tiles;
  const int64_t s0 = 2 * int64_t(q);
  int64_t m0, n0;
  {
    const int per_band = kBandRows * p.tiles_n;
    const int band = tile / per_band, in_band = tile % per_band;
    const int rows_left = p.tiles_m - band * kBandRows;
    const int band_rows = rows_left < kBandRows ? rows_left : kBandRows;
    m0 = int64_t(band * kBandRows + in_band % band_rows) * kPairTile;
    n0 = int64_t(in_band / band_rows) * kPairTile;
  }
  unsigned tag = 0;
  if (threadIdx.x == 0)
    tag = __hip_atomic_load(p.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  const int rb0 = pair_region_first(q, ng), rb1 = pair_region_first(q + 1, ng);
  const int nitems = (rb1 - rb0) * 128;

  // bias: this lane's columns of the bias operand (rows wm + 32 i + lane % 32
  // of a, or columns wn + 32 j + lane % 32 of b; k half lane / 32)
  const int tile_m = static_cast<int>(m0 / kPairTile), tile_n = static_cast<int>(n0 / kPairTile);
  const int blim = bias_limit(BOP == 1 ? p.M : p.N, BOP == 1 ? m0 : n0);
  float bcs[3] = {0.f, 0.f, 0.f}, bsq = 0.f;
  auto fhook = [&](int kt, int ks, const dma::Frags<G>& f) {
    if constexpr (BOP == 1) {
      if (kt % p.tiles_n == tile_n && (wl & 1) == ks) {
#pragma unroll
        for (int i = 0; i < 3; ++i)
          bias_frag<DT>(f.a[i], bcs[i], bsq, wm + 32 * i + (lane & 31), blim);
      }
    } else if constexpr (BOP == 2) {
      if (kt % p.tiles_m == tile_m && (wl >> 1) == ks) {
#pragma unroll
        for (int j = 0; j < 3; ++j)
          bias_frag<DT>(f.b[j], bcs[j], bsq, wn + 32 * j + (lane & 31), blim);
      }
    }
  };

  // ---- 1. the two products
  f32x16 acc[3][3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  {
    dma::FragOffsets<G> fo;
    fo.init(half * kPairTile + wm, half * kPairTile + wn);
    dma::PairJob<G> job;
    job.init(p.a + s0 * p.sab, p.lda, p.sab, p.b + s0 * p.sbb, p.ldb, p.sbb, p.K, m0, n0);
    dma::gemm_pipe<DT, G, S>(job, static_cast<int>(p.K / G::BK), fo, stages, acc, dma::NoHook(),
                             fhook);
  }
  {
    // rows/columns past M/N may hold the next row's values: left out of the norm
    const int64_t rl = p.M - m0, cl = p.N - n0;
    const int rlim = rl < kPairTile ? static_cast<int>(rl) : kPairTile;
    const int clim = cl < kPairTile ? static_cast<int>(cl) : kPairTile;
    float sq = 0.f;
    if (rlim == kPairTile && clim == kPairTile) {
#pragma unroll
      for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) sq = __builtin_fmaf(acc[i][j][r], acc[i][j][r], sq);
    } else {
#pragma unroll
      for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const bool ncol = acc_col(wn, j, lane) < clim;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float v = ncol && acc_row(wm, i, lane, r) < rlim ? acc[i][j][r] : 0.f;
            sq = __builtin_fmaf(v, v, sq);
          }
        }
    }
    sq = wave_sum_dpp(sq);
    if (lane == 0) red[wave] = sq;
    if (threadIdx.x == 0) {
      tag_s = tag;
      bbad = 0;
    }
    __syncthreads();
    tag = tag_s;
    // the two samples' partials of this tile, each one 64-bit store of the
    // value and the launch's tag (complemented: a pattern no fp32 or bf16 data
    // left in the workspace carries), so that both become visible together
    if (threadIdx.x < 2) {
      const float* r4 = red + 4 * threadIdx.x;
      const float v = (r4[0] + r4[1]) + (r4[2] + r4[3]);
      __hip_atomic_store(p.tagged + (s0 + threadIdx.x) * p.tiles + tile,
                         (uint64_t(~tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if constexpr (BIAS) {
    // the bias's column sums: lanes l and l + 32 hold one column's two k
    // halves; the two waves of a sample that share a fragment (one k-step
    // each) are added in wave order through st0 ([sample][wave][192], free:
    // gemm_pipe ended on a barrier).  Then one tagged word per (column,
    // sample) and one per (sample, tile) for the squares.
    float* colp = reinterpret_cast<float*>(st0);
    const int ws = BOP == 1 ? (wl & 1) : (wl >> 1);
    const int cl0 = BOP == 1 ? wm : wn;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const float v = bcs[i] + __shfl_xor(bcs[i], 32, kWave);
      if (lane < 32) colp[(half * 2 + ws) * kPairTile + cl0 + 32 * i + lane] = v;
    }
    const float q = wave_sum_dpp(bsq);
    if (lane == 0) bred[wave] = q;
    __syncthreads();
    const int own = BOP == 1 ? tile_m : tile_n, oth = BOP == 1 ? tile_n : tile_m;
    const int P = BOP == 1 ? p.tiles_n : p.tiles_m;
    for (int r = threadIdx.x; r < 2 * kPairTile; r += kWideThreads) {
      const int h = r / kPairTile, c = r % kPairTile;
      const float v = colp[(h * 2) * kPairTile + c] + colp[(h * 2 + 1) * kPairTile + c];
      const int64_t word = ((int64_t(own) * kPairTile + c) * p.B + s0 + h) * P + oth;
      __hip_atomic_store(p.bias_tagged + word, (uint64_t(~tag) << 32) | __float_as_uint(v),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (threadIdx.x < 2) {
      const float* q4 = bred + 4 * threadIdx.x;
      const float v = (q4[0] + q4[1]) + (q4[2] + q4[3]);
      __hip_atomic_store(p.bias_sq_tagged + (s0 + threadIdx.x) * p.tiles + tile,
                         (uint64_t(~tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();  // (st0 is staged into next)
  }

  // The launch epoch (the next launch's tags) advances once every workgroup
  // has read it: the last one to count itself here advances it and resets the
  // self-clearing counter.
  unsigned* const start_cnt = p.group_cnt + p.tiles;
  unsigned started = 0;
  if (threadIdx.x == 0)
    started = __hip_atomic_fetch_add(start_cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // The finish stores chunks of 8 consecutive outputs of one row: chunk ch
  // of the region is row (ch / 4) % 32, columns 8 * (ch % 4) .. + 7 of block
  // rb0 + ch / 128; chunk_pos gives its first output.
  const int nchunks = (rb1 - rb0) * 128;
  auto chunk_pos = [&](int ch, int64_t& row, int64_t& col) {
    const int bid = rb0 + (ch >> 7), r = (ch >> 2) & 31;
    const int w = bid / 9, ij = bid % 9;
    row = m0 + (w >> 1) * 96 + 32 * (ij / 3) + r;
    col = n0 + (w & 1) * 96 + 32 * (ij % 3) + 8 * (ch & 3);
  };
  const NoiseSrc nz = p.noise.resolved();
  const bool pre_noise = nz.on() && nz.z == nullptr && p.N % 4 == 0;
  f32x4* zpre = reinterpret_cast<f32x4*>(st2);  // the two Philox blocks of each chunk

  if (threadIdx.x == 0 && started + 1 == unsigned(p.nwg)) {
    __hip_atomic_store(start_cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_fetch_add(p.epoch, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // ---- 2. the clip factors: wave w < 2 polls sample s0 + w's partials (all tiles,
  // written by the pair's workgroups) until each carries this launch's tag,
  // then sums them in tile order; a bounded wait
  if (wave < 2) {
    float C = p.C, clamp = p.clamp;
    if (p.clip_args_dev != nullptr) {
      C = p.clip_args_dev[0];
      clamp = p.clip_args_dev[1];
    }
    const int64_t s = s0 + wave;
    const uint64_t* part = p.tagged + s * p.tiles;
    const uint32_t want = ~tag;
    float a = 0.f;
    bool bad = false;
    for (int t0 = 0; t0 < p.tiles && !bad; t0 += kWave) {
      const int t = t0 + lane;
      uint64_t v = uint64_t(want) << 32;
      for (unsigned spins = 0;; ++spins) {
        if (spins >= p.spin_limit) {
          bad = true;
          break;
        }
        if (t < p.tiles) v = __hip_atomic_load(part + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__all(uint32_t(v >> 32) == want)) break;
        __builtin_amdgcn_s_sleep(2);
      }
      a += __uint_as_float(uint32_t(v));
    }
    a = wave_sum_dpp(a);
    if (lane == 0) {
      if (bad) expire(p.err, p.poison, tag);
      const float n = bad ? __builtin_nanf("") : sqrtf(a);
      const float cf = bad ? n : clip_factor(n, C, clamp);
      fac[wave] = cf;
      bad2[wave] = bad;
      if (tile == 0) {  // one writer per sample
        if (p.norms_out) p.norms_out[s] = n;
        if (p.factors_out) p.factors_out[s] = cf;
      }
    }
  }
  __syncthreads();
  bool poisoned = bad2[0] != 0 || bad2[1] != 0;

  // ---- 3./4. S = c0 G0 + c1 G1, one row i of blocks at a time.  Waves w and
  // w + 4 hold the same blocks; for block (i, j) one of them (the stager)
  // puts its scaled block in LDS ([wave][j][register quad][lane], 16-byte
  // words; rows alternate between st0 and st2) and the other (the adder,
  // alternating with the block index) adds its own, then keeps the sum (own
  // region, st1: [block][half][lane][8]) or publishes it (bf16).  Row i + 1
  // is staged while row i is added.
  const float cmine = fac[half];
  f32x4* const stg[2] = {reinterpret_cast<f32x4*>(st0), reinterpret_cast<f32x4*>(st2)};
  f32x4* own = reinterpret_cast<f32x4*>(st1);
  const int slot_bytes = p.slot_blocks * kWideBlockBytes;
  {
    const CoherentSpan slot(reinterpret_cast<const float*>(p.slots + int64_t(L) * slot_bytes),
                            static_cast<uint32_t>(slot_bytes));
    auto stage = [&](auto i_c, f32x4* buf) {
      constexpr int i = decltype(i_c)::value;
#pragma unroll
      for (int j = 0; j < 3; ++j)
        if (((i * 3 + j) & 1) != half) {
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4)
            buf[((wl * 3 + j) * 4 + r4) * 64 + lane] =
                f32x4{cmine * acc[i][j][4 * r4], cmine * acc[i][j][4 * r4 + 1],
                      cmine * acc[i][j][4 * r4 + 2], cmine * acc[i][j][4 * r4 + 3]};
        }
    };
    auto add = [&](auto i_c, const f32x4* buf) {
      constexpr int i = decltype(i_c)::value;
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        if (((i * 3 + j) & 1) != half) continue;
        const int bid = wl * 9 + i * 3 + j;
        float v[16];
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const f32x4 o = buf[((wl * 3 + j) * 4 + r4) * 64 + lane];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            v[4 * r4 + e] = __builtin_fmaf(cmine, acc[i][j][4 * r4 + e], o[e]);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (bid >= rb0 && bid < rb1) {
            f32x4* o = own + (((bid - rb0) * 2 + h) * 64 + lane) * 2;
            o[0] = f32x4{v[8 * h], v[8 * h + 1], v[8 * h + 2], v[8 * h + 3]};
            o[1] = f32x4{v[8 * h + 4], v[8 * h + 5], v[8 * h + 6], v[8 * h + 7]};
          } else {
            u32x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = BF16::pack2(v[8 * h + 2 * e], v[8 * h + 2 * e + 1]);
            slot.store4(
                static_cast<uint32_t>((slot_block(bid, rb0, rb1) * 2 + h) * 1024 + lane * 16),
                __builtin_bit_cast(f32x4, w));
          }
        }
      }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    stage(I0{}, stg[0]);
    __syncthreads();
    stage(I1{}, stg[1]);
    add(I0{}, stg[0]);
    __syncthreads();
    stage(I2{}, stg[0]);
    add(I1{}, stg[1]);
    __syncthreads();
    add(I2{}, stg[0]);
  }

  // the noise of the region (st2 is free again), drawn while the published
  // blocks drain
  if (pre_noise) {
#pragma unroll 1
    for (int ch = threadIdx.x; ch < nchunks; ch += kWideThreads) {
      int64_t row, col;
      chunk_pos(ch, row, col);
#pragma unroll 1
      for (int u = 0; u < 2; ++u) {
        float blk[4];
        nz.block((row * p.N + col) / 4 + u, blk);
        zpre[ch * 2 + u] = f32x4{blk[0], blk[1], blk[2], blk[3]};
      }
    }
  }

  // ---- 5. the tile's workgroups wait for each other
  unsigned* cnt = p.group_cnt + tile;
  const unsigned garr = grid_arrive(cnt);
  poisoned = grid_wait(cnt, unsigned(ng), garr, p.err, nullptr, p.poison, tag, p.spin_limit, &flag,
                       0, 2) || poisoned;

  // ---- 6. finish.  Item it of the region (block rb0 + it/128, half
  // (it/64)%2, lane it%64: rows {0..3, 8..11} + 16 half + 4 (lane/32) of
  // column lane%32 of the block) is the sum of the pairs' chunks in pair
  // order; the sums go to st0 in row-major blocks ([block][32 rows][32]),
  // from which each thread stores chunks of 8 consecutive outputs of a row:
  // out = out_scale * sum + noise_scale * z.
  const int64_t slot_stride = int64_t(p.tiles) * slot_bytes;  // between pairs of one tile
  const char* const slots_tile = p.slots + int64_t(tile) * slot_bytes;
  float* const rows = reinterpret_cast<float*>(st0);
  auto slot_load = [&](int qq, int it) -> u32x4 {
    const int bid = rb0 + (it >> 7), h = (it >> 6) & 1, l = it & 63;
    const CoherentSpan sl(reinterpret_cast<const float*>(slots_tile + qq * slot_stride),
                          static_cast<uint32_t>(slot_bytes));
    const int sb = slot_block(bid, pair_region_first(qq, ng), pair_region_first(qq + 1, ng));
    return __builtin_bit_cast(u32x4, sl.load4(static_cast<uint32_t>((sb * 2 + h) * 1024 + l * 16)));
  };
  auto add_own = [&](float (&v)[8], int it) {
    const int lb = it >> 7, h = (it >> 6) & 1, l = it & 63;
    const f32x4* o = own + ((lb * 2 + h) * 64 + l) * 2;
    const f32x4 lo = o[0], hi = o[1];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] += lo[e];
      v[4 + e] += hi[e];
    }
  };
  auto add_bf16 = [&](float (&v)[8], const u32x4& w) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      v[2 * e] += __uint_as_float(w[e] << 16);
      v[2 * e + 1] += __uint_as_float(w[e] & 0xffff0000u);
      v[4 + 2 * e] += __uint_as_float(w[2 + e] << 16);
      v[4 + 2 * e + 1] += __uint_as_float(w[2 + e] & 0xffff0000u);
    }
  };
  auto put_rows = [&](int it, const float (&v)[8]) {
    const int lb = it >> 7, h = (it >> 6) & 1, l = it & 63;
    float* b = rows + lb * 1024 + (16 * h + 4 * (l >> 5)) * 32 + (l & 31);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      b[e * 32] = v[e];
      b[(8 + e) * 32] = v[4 + e];
    }
  };
  constexpr int R = (kPairRegionMax * 128 + kWideThreads - 1) / kWideThreads;
  static_assert(R == 3, "three rounds of items per thread at most");
  if (ng <= kPairFast) {
    // every chunk of every item of this thread in flight at once (at most
    // R x (kPairFast - 1) loads), then the sums
    u32x4 w[R][kPairFast];
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int it = threadIdx.x + k * kWideThreads;
      if (it < nitems) {
#pragma unroll
        for (int qq = 0; qq < kPairFast; ++qq)
          if (qq < ng && qq != q) w[k][qq] = slot_load(qq, it);
      }
    }
#pragma unroll 1
    for (int k = 0; k < R; ++k) {
      const int it = threadIdx.x + k * kWideThreads;
      if (it >= nitems) break;
      float v[8] = {};
      // (round k's chunks through selects: the register arrays stay static)
#pragma unroll
      for (int qq = 0; qq < kPairFast; ++qq) {
        if (qq >= ng) break;
        if (qq == q) add_own(v, it);
        else add_bf16(v, k == 0 ? w[0][qq] : k == 1 ? w[1][qq] : w[2][qq]);
      }
      put_rows(it, v);
    }
  } else {
#pragma unroll 1
    for (int it = threadIdx.x; it < nitems; it += kWideThreads) {
      float v[8] = {};
      // chunks in pair order, kPairFast loads in flight at a time
#pragma unroll 1
      for (int qb = 0; qb < ng; qb += kPairFast) {
        u32x4 w[kPairFast];
#pragma unroll
        for (int u = 0; u < kPairFast; ++u)
          if (qb + u < ng && qb + u != q) w[u] = slot_load(qb + u, it);
#pragma unroll
        for (int u = 0; u < kPairFast; ++u) {
          if (qb + u >= ng) break;
          if (qb + u == q) add_own(v, it);
          else add_bf16(v, w[u]);
        }
      }
      put_rows(it, v);
    }
  }
  __syncthreads();
  const int oes = p.out_dtype == FDP_F32 ? 4 : 2;
  const bool vec8 = reinterpret_cast<uintptr_t>(p.out) % (8 * oes) == 0 && p.ldo % 8 == 0;
#pragma unroll 1
  for (int ch = threadIdx.x; ch < nchunks; ch += kWideThreads) {
    int64_t row, col;
    chunk_pos(ch, row, col);
    const f32x4* src = reinterpret_cast<const f32x4*>(rows + (ch >> 7) * 1024 + ((ch >> 2) & 31) * 32 +
                                                      8 * (ch & 3));
    float o[8];
    {
      const f32x4 lo = src[0], hi = src[1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] = lo[e] * p.out_scale;
        o[4 + e] = hi[e] * p.out_scale;
      }
    }
    if (nz.on()) {
      if (pre_noise) {
        const f32x4 z0 = zpre[ch * 2], z1 = zpre[ch * 2 + 1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[e] += p.noise_scale * z0[e];
          o[4 + e] += p.noise_scale * z1[e];
        }
      } else {
        // an injected tensor, or rows of N % 4 != 0 outputs: element by element
#pragma unroll 1
        for (int e = 0; e < 8; ++e) {
          const float ze = (row < p.M && col + e < p.N) ? nz.at(row * p.N + col + e) : 0.f;
#pragma unroll
          for (int d = 0; d < 8; ++d) o[d] += d == e ? p.noise_scale * ze : 0.f;
        }
      }
    }
    if (poisoned) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = __builtin_nanf("");
    }
    if (row >= p.M) continue;
    const int64_t at = row * p.ldo + col;
    if (vec8 && col + 8 <= p.N) {
      if (p.out_dtype == FDP_F32) {
        f32x4* d = reinterpret_cast<f32x4*>(static_cast<float*>(p.out) + at);
        d[0] = f32x4{o[0], o[1], o[2], o[3]};
        d[1] = f32x4{o[4], o[5], o[6], o[7]};
      } else {
        u32x4 pk;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          pk[e] = p.out_dtype == FDP_BF16 ? BF16::pack2(o[2 * e], o[2 * e + 1])
                                          : F16::pack2(o[2 * e], o[2 * e + 1]);
        *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p.out) + at) = pk;
      }
    } else {
#pragma unroll 1
      for (int e = 0; e < 8; ++e)
        if (col + e < p.N) store_from_f32(p.out, at + e, p.out_dtype, o[e]);
    }
  }

  // ---- 7. the bias: outputs [L * per, (L + 1) * per) of len, eight threads
  // each.  Output c is the sum over the J = B * P partials (sample s, partial
  // q; word j = s * P + q) of c'_s * part[c][s][q]: thread u of the eight takes
  // words u, u + 8, ... in that order, and the eight sums are added in a fixed
  // tree.  The clip factors c'_s are formed by every workgroup from all
  // samples' squares (wave w: samples w, w + 8, ...).  Every word was published
  // right after the products; the first words are requested before the
  // squares, so that one round trip brings both.  The polls are bounded like
  // the others.
  if constexpr (BIAS) {
    const int64_t len = BOP == 1 ? p.M : p.N;
    const int P = BOP == 1 ? p.tiles_n : p.tiles_m;
    const int nb = static_cast<int>(p.B);
    const int J = nb * P;
    const uint32_t want = ~tag;
    const int64_t per = (len + p.nwg - 1) / p.nwg;
    const int64_t lo = int64_t(L) * per, hi = lo + per < len ? lo + per : len;
    const int sub = threadIdx.x & 7;
    uint64_t w8[8];
    auto issue = [&](int64_t m, int j0) {
      const uint64_t* words = p.bias_tagged + m * J;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + sub + 8 * u;
        w8[u] = m < hi && j < J
                    ? __hip_atomic_load(words + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                    : uint64_t(want) << 32;
      }
    };
    issue(lo + (threadIdx.x >> 3), 0);
    {
      float C = p.C, clamp = p.clamp;
      if (p.clip_args_dev != nullptr) {
        C = p.clip_args_dev[0];
        clamp = p.clip_args_dev[1];
      }
      for (int sm = wave; sm < nb; sm += kWideThreads / kWave) {
        const uint64_t* part = p.bias_sq_tagged + int64_t(sm) * p.tiles;
        float a = 0.f;
        bool bad = false;
        for (int t0 = 0; t0 < p.tiles && !bad; t0 += kWave) {
          const int t = t0 + lane;
          uint64_t v = uint64_t(want) << 32;
          for (unsigned spins = 0;; ++spins) {
            if (spins >= p.spin_limit) {
              bad = true;
              break;
            }
            if (t < p.tiles) v = __hip_atomic_load(part + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (__all(uint32_t(v >> 32) == want)) break;
            __builtin_amdgcn_s_sleep(2);
          }
          a += __uint_as_float(uint32_t(v));
        }
        a = wave_sum_dpp(a);
        if (lane == 0) {
          const float n = bad || poisoned ? __builtin_nanf("") : sqrtf(a);
          const float cf = bad || poisoned ? n : clip_factor(n, C, clamp);
          bfac[sm] = cf;
          if (bad) {
            bbad = 1;
            expire(p.err, p.poison, tag);
          }
          if (L == 0) {  // one writer
            if (p.bias_norms) p.bias_norms[sm] = n;
            if (p.bias_factors) p.bias_factors[sm] = cf;
          }
        }
      }
    }
    __syncthreads();
    for (int64_t mb = lo; mb < hi; mb += kWideThreads / 8) {
      const int64_t m = mb + (threadIdx.x >> 3);
      const uint64_t* words = p.bias_tagged + m * J;
      float v = 0.f;
      bool bad = false;
#pragma unroll 1
      for (int j0 = 0; j0 < J; j0 += 64) {
        if (mb != lo || j0 != 0) issue(m, j0);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int j = j0 + sub + 8 * u;
          // (a word not yet visible is polled again, boundedly)
          for (unsigned spins = 0; uint32_t(w8[u] >> 32) != want; ++spins) {
            if (spins >= p.spin_limit) {
              bad = true;
              w8[u] = uint64_t(want) << 32;
              break;
            }
            __builtin_amdgcn_s_sleep(2);
            w8[u] = __hip_atomic_load(words + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          if (m < hi && j < J) v += bfac[j / P] * __uint_as_float(uint32_t(w8[u]));
        }
      }
      if (bad && bbad == 0 && !poisoned) expire(p.err, p.poison, tag);
      if (bad || bbad != 0 || poisoned) v = __builtin_nanf("");
      v += __shfl_xor(v, 1, kWave);
      v += __shfl_xor(v, 2, kWave);
      v += __shfl_xor(v, 4, kWave);
      if (sub == 0 && m < hi) {
        v *= p.bias_scale;
        if (p.bias_noise.on()) v += p.bias_noise_scale * p.bias_noise.at(m);
        store_from_f32(p.bias_out, m, p.bias_dtype, v);
      }
    }
  }
}

// Tile orientation and workspace of the wide schedule for a problem: 384x192
// (WGM = 4) or 192x384 (WGM = 2) output tiles, whichever wastes fewer
// outputs; applicable when every product gets a CU of its own, the products
// fill at least `min_fill` of the device, and the row strides keep a
// sample's operand under 2^31 bytes (32-bit buffer records).

struct WidePlan {
  // one sample per workgroup: wgm 4 (384x192 tiles), 2 (192x384), 0 (not applicable)
  int wgm;
  int tiles_m, tiles_n, tiles, nwg;
  int slot_blocks;
  // two samples per workgroup (192x192 tiles, wgrad_pair_kernel): pair 0 = not applicable
  int pair;
  int pair_tiles_m, pair_tiles_n, pair_tiles, pair_nwg;
  int pair_slot_blocks;
  size_t partial_bytes, slot_bytes;       // the larger of the two layouts'
  size_t bias_part_bytes, bias_sq_bytes;  // the bias of a or b, the larger of the two
                                          // layouts' (reserved whether asked or not)
  bool any() const { return wgm != 0 || pair != 0; }
};
// The paired layout also needs whole k-tiles and both samples of a pair
// inside one 32-bit buffer record ((sab + K * lda) * 2 bytes): checked here for
// contiguous operands, by the caller for the strides of the call.
inline bool pair_records_fit(int64_t K, int64_t ld, int64_t ds) {
  return fits_record(K, ld, ds);
}
inline WidePlan wide_plan(int64_t B, int64_t K, int64_t M, int64_t N, int64_t lda, int64_t ldb,
                          int cus, double min_fill) {
  WidePlan w{};
  if (!fits_record(K, lda) || !fits_record(K, ldb)) return w;
  const double fill = double(M) * double(N) * double(B) / (double(cus) * 73728.0);
  if (fill < min_fill) return w;
  int64_t best_tiles = 0;
  for (int wgm : {4, 2}) {
    const int64_t tm = 96 * wgm, tn = 96 * (8 / wgm);
    const int64_t t = ((M + tm - 1) / tm) * ((N + tn - 1) / tn);
    if (best_tiles == 0 || t < best_tiles) {
      best_tiles = t;
      w.wgm = wgm;
      w.tiles_m = static_cast<int>((M + tm - 1) / tm);
      w.tiles_n = static_cast<int>((N + tn - 1) / tn);
    }
  }
  w.tiles = static_cast<int>(best_tiles);
  const int64_t units = best_tiles * B;
  if (units > cus || B < 2 || B > kWideBlocks) {
    w.wgm = 0;
  } else {
    w.nwg = static_cast<int>(units);
    w.slot_blocks = kWideBlocks - static_cast<int>(kWideBlocks / B);
    w.partial_bytes = sizeof(float) * size_t(units);
    w.slot_bytes = size_t(units) * size_t(w.slot_blocks) * kWideBlockBytes;
    // [tiles_own, W, B, tiles_other] with W <= 384 for either operand
    w.bias_part_bytes = sizeof(float) * size_t(B) * w.tiles_m * w.tiles_n * 384;
    w.bias_sq_bytes = sizeof(float) * size_t(units);
  }
  const int64_t ptm = (M + kPairTile - 1) / kPairTile, ptn = (N + kPairTile - 1) / kPairTile;
  const int64_t punits = ptm * ptn * (B / 2);
  if (B % 2 == 0 && B >= kPairMinB && B <= 2 * kPairBlocks && K % PairGeom::BK == 0 &&
      ptm * ptn + 1 <= kGroupMax && punits <= cus && pair_records_fit(K, lda, K * lda) &&
      pair_records_fit(K, ldb, K * ldb)) {
    w.pair = 1;
    w.pair_tiles_m = static_cast<int>(ptm);
    w.pair_tiles_n = static_cast<int>(ptn);
    w.pair_tiles = static_cast<int>(ptm * ptn);
    w.pair_nwg = static_cast<int>(punits);
    const int ng = static_cast<int>(B / 2);
    w.pair_slot_blocks = kPairBlocks - kPairBlocks / ng;
    const size_t pb = sizeof(uint64_t) * size_t(B) * w.pair_tiles;
    const size_t sb = size_t(punits) * size_t(w.pair_slot_blocks) * kWideBlockBytes;
    // bias: [tiles_own * 192][B][P] words with tiles_own * P = the tile count
    const size_t bp = sizeof(uint64_t) * size_t(kPairTile) * size_t(B) * w.pair_tiles;
    const size_t bq = sizeof(uint64_t) * size_t(B) * w.pair_tiles;
    if (pb > w.partial_bytes) w.partial_bytes = pb;
    if (sb > w.slot_bytes) w.slot_bytes = sb;
    if (bp > w.bias_part_bytes) w.bias_part_bytes = bp;
    if (bq > w.bias_sq_bytes) w.bias_sq_bytes = bq;
  }
  return w;
}

// wgm 4 / 2: the one-sample kernel in that orientation; wgm 1: the paired
// kernel.
template <class DT>
hipError_t launch_wide_t(const WideArgs& a, int wgm, bool plain, hipStream_t s) {
  const void* fns[2][3] = {
      {reinterpret_cast<const void*>(&wgrad_wide_kernel<DT, 4, 2, 0>),
       reinterpret_cast<const void*>(&wgrad_wide_kernel<DT, 4, 2, 1>),
       reinterpret_cast<const void*>(&wgrad_wide_kernel<DT, 4, 2, 2>)},
      {reinterpret_cast<const void*>(&wgrad_wide_kernel<DT, 2, 4, 0>),
       reinterpret_cast<const void*>(&wgrad_wide_kernel<DT, 2, 4, 1>),
       reinterpret_cast<const void*>(&wgrad_wide_kernel<DT, 2, 4, 2>)}};
  const void* pairs[3] = {reinterpret_cast<const void*>(&wgrad_pair_kernel<DT, 0>),
                          reinterpret_cast<const void*>(&wgrad_pair_kernel<DT, 1>),
                          reinterpret_cast<const void*>(&wgrad_pair_kernel<DT, 2>)};
  if (a.bias_op < 0 || a.bias_op > 2) return hipErrorInvalidValue;
  const void* fn = wgm == 1 ? pairs[a.bias_op] : fns[wgm == 4 ? 0 : 1][a.bias_op];
  if (host::occupancy(fn, kWideThreads, 0) < 1) return hipErrorNotSupported;
  WideArgs c = a;
  void* params[] = {&c};
  return plain ? hipLaunchKernel(fn, dim3(a.nwg), dim3(kWideThreads), params, 0, s)
               : hipLaunchCooperativeKernel(fn, dim3(a.nwg), dim3(kWideThreads), params, 0, s);
}

hipError_t launch_wide_bf16(const WideArgs& a, int wgm, bool plain, hipStream_t s);
hipError_t launch_wide_f16(const WideArgs& a, int wgm, bool plain, hipStream_t s);

}  // namespace wg
}  // namespace fdp
