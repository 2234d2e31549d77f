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
  // out_scale, noise, store.  Each 4-row group of the item is transposed in
  // its quad of lanes: lane k then holds row k's 4 consecutive outputs, one
  // vector store (and the row layout of the Philox draw).
  auto finish = [&](int it, const float (&v)[8]) {
    int64_t mr, nc;
    item_pos(it, mr, nc);
    const int64_t n4 = nc & ~int64_t(3);
#pragma unroll 1
    for (int grp = 0; grp < 2; ++grp) {
      float src[4], o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) src[k] = (grp == 0 ? v[k] : v[4 + k]) * p.out_scale;
      quad_transpose(src, o);
      const int64_t row = mr + 8 * grp + (lane & 3);
      if (noisy) {
        float z[4];
        if (pre_noise) {
          const f32x4 zz = zpre[it * 2 + grp];
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

// Tile orientation and workspace of the wide schedule for a problem: 384x192
// (WGM = 4) or 192x384 (WGM = 2) output tiles, whichever wastes fewer
// outputs; applicable when every product gets a CU of its own, the products
// fill at least `min_fill` of the device, and the row strides keep a
// sample's operand under 2^31 bytes (32-bit buffer records).

struct WidePlan {
  int wgm;  // 4: 384x192, 2: 192x384, 0: not applicable
  int tiles_m, tiles_n, tiles, nwg;
  int slot_blocks;
  size_t partial_bytes, slot_bytes;
  size_t bias_part_bytes, bias_sq_bytes;  // the bias of a or b (reserved whether asked or not)
};
inline WidePlan wide_plan(int64_t B, int64_t K, int64_t M, int64_t N, int64_t lda, int64_t ldb,
                          int cus, double min_fill) {
  WidePlan w{};
  if (K * lda * 2 >= (int64_t(1) << 31) || K * ldb * 2 >= (int64_t(1) << 31)) return w;
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
  const double fill = double(M) * double(N) * double(B) / (double(cus) * 73728.0);
  if (units > cus || fill < min_fill || B < 2 || B > kWideBlocks) {
    w.wgm = 0;
    return w;
  }
  w.nwg = static_cast<int>(units);
  w.slot_blocks = kWideBlocks - static_cast<int>(kWideBlocks / B);
  w.partial_bytes = sizeof(float) * size_t(units);
  w.slot_bytes = size_t(units) * size_t(w.slot_blocks) * kWideBlockBytes;
  // [tiles_own, W, B, tiles_other] with W <= 384 for either operand
  w.bias_part_bytes = sizeof(float) * size_t(B) * w.tiles_m * w.tiles_n * 384;
  w.bias_sq_bytes = sizeof(float) * size_t(units);
  return w;
}

template <class DT>
hipError_t launch_wide_t(const WideArgs& a, int wgm, bool plain, hipStream_t s) {
  const void* fns[2][3] = {
      {reinterpret_cast<const void*>(&wgrad_wide_kernel<DT, 4, 2, 0>),
       reinterpret_cast<const void*>(&wgrad_wide_kernel<DT, 4, 2, 1>),
       reinterpret_cast<const void*>(&wgrad_wide_kernel<DT, 4, 2, 2>)},
      {reinterpret_cast<const void*>(&wgrad_wide_kernel<DT, 2, 4, 0>),
       reinterpret_cast<const void*>(&wgrad_wide_kernel<DT, 2, 4, 1>),
       reinterpret_cast<const void*>(&wgrad_wide_kernel<DT, 2, 4, 2>)}};
  if (a.bias_op < 0 || a.bias_op > 2) return hipErrorInvalidValue;
  const void* fn = fns[wgm == 4 ? 0 : 1][a.bias_op];
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
