// Two-pass clipped weight gradient for layers whose per-sample products do
// not fit the register file of the resident grid (more 128x128 output tiles
// than co-resident workgroups):
//
//   norm pass  ||G_b||_F^2 = sum_{t,s} (g_t . g_s)(x_t . x_s)
//              (gram_norm_kernel): the Frobenius inner product of the two
//              per-sample Gram matrices g_b g_b^T and x_b x_b^T, [T, T] each,
//              over the upper triangle of 128 x 128 Gram tiles (off-diagonal
//              tiles count twice).  Per sample this is ~T^2/2 (M + N)
//              multiply-adds instead of the T M N of forming G_b, so it is
//              chosen when that is smaller.
//   sum pass   out = out_scale sum_b c_b G_b + noise_scale z (clipsum_kernel):
//              one long contraction per output tile over every sample's T
//              rows, streamed through an LDS ring; the accumulator is
//              rescaled by c_prev / c_b where sample b starts, so that it
//              always holds sum c_j G_j / c_b and the per-sample product is
//              never formed on its own.
//
// Both run on the LDS-DMA MFMA core of gemm_dma.hpp.  The Gram operands are
// rows of g_b / x_b with the contraction axis contiguous, read as 16-byte
// MFMA fragments (ds_read_b128) from an XOR-swizzled row-major LDS tile; the
// sum pass reads the [T, M] / [T, N] operands with transposing LDS reads.
#pragma once

#include "wgrad_core.hpp"

namespace fdp {
namespace wg {

// ------------------------------------------------------------ [R, K] operand
// An R x 64 tile of a row-major operand whose contraction axis k is
// contiguous: R rows of 128 bytes (8 chunks of 16 bytes).  Chunk c of row r
// sits at physical chunk c ^ rswz(r), which spreads both the DMA writes and
// the fragment reads (32 consecutive rows, one chunk each) over the banks.
__device__ __forceinline__ int rswz(int r) { return (r ^ (r >> 3)) & 7; }

template <int L>
struct OperandRK {
  u32x4 rsrc;        // raw buffer over the tile's first row .. the sample's last row
  uint32_t voff[L];  // byte offsets of this thread's loads for k-tile 0
  // base: first row of the tile; ld: row stride (elements); rows: rows left
  // in the sample (rows at or past it read as zero).
  __device__ inline void init(const uint16_t* base, int64_t ld, int64_t rows) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    retarget(base, ld, rows);
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const int slot = (wave * L + j) * 64 + lane;
      const int r = slot >> 3;
      const int c = (slot & 7) ^ rswz(r);
      voff[j] = static_cast<uint32_t>((int64_t(r) * ld + 8 * c) * 2);
    }
  }
  __device__ __forceinline__ void retarget(const uint16_t* base, int64_t ld, int64_t rows) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    const int64_t bytes = rows > 0 ? rows * ld * 2 : 0;
    rsrc = u32x4{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xffffu,
                 static_cast<uint32_t>(bytes), dma::kRsrcWord3};
  }
  // k-tile kt (64 k-values, 128 bytes further along every row)
  __device__ __forceinline__ void issue(FDP_LDS char* tile, int kt) const {
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(tile)) + wave * L * 1024;
    const uint32_t add = 128u * static_cast<uint32_t>(kt);
    u32x4 r;
#pragma unroll
    for (int w = 0; w < 4; ++w) r[w] = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(rsrc[w]));
#pragma unroll
    for (int j = 0; j < L; ++j) {
      uint32_t saved;
      asm volatile(
          "s_mov_b32 %0, m0\n\t"
          "s_mov_b32 m0, %1\n\t"
          "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
          "s_mov_b32 m0, %0"
          : "=&s"(saved)
          : "s"(lds + j * 1024), "v"(voff[j] + add), "s"(r)
          : "memory");
    }
  }
};

// Byte offset of this lane's 16-byte MFMA fragment (rows w0 + 32i + lane%32,
// k-values 8*(lane/32) .. +7 of k-step 0) in a 128-byte-row tile; k-step ks
// is the same offset XOR (ks << 5).
__device__ __forceinline__ uint32_t rk_frag_off(int w0, int i) {
  const int lane = threadIdx.x & 63;
  const int r = w0 + 32 * i + (lane & 31);
  return static_cast<uint32_t>(r * 128 + (((lane >> 5) ^ rswz(r)) << 4));
}

__device__ __forceinline__ uint4 read_frag_b128(const FDP_LDS char* tile, uint32_t off) {
  const u32x4 w = *reinterpret_cast<const FDP_LDS u32x4*>(tile + off);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// ---------------------------------------------------------------- Gram norm
// Work item (b, ti, tj), ti <= tj: 128-row tiles ti, tj of sample b.  Unit 0
// is the g-Gram tile over the M features, unit 1 the x-Gram tile over the N
// features; the item's partial is w * sum(Gg .* Gx), w = 1 on the diagonal, 2
// off it.  Requires M % 64 == 0 and N % 64 == 0 (no partial k-tiles).
constexpr int kGramT = 128;

struct GramArgs {
  const uint16_t* a;  // g: [B] x [T, M], row stride lda, sample stride sab
  const uint16_t* b;  // x: [B] x [T, N]
  int64_t B, T, M, N, sab, lda, sbb, ldb;
  int nt;             // 128-row tiles per sample
  int per_sample;     // nt (nt + 1) / 2 items
  int64_t items;      // B * per_sample
  float* partials;    // [B, per_sample]
};

__device__ __forceinline__ void gram_item(int r, int nt, int& ti, int& tj) {
  int i = 0;
  while (r >= nt - i) {
    r -= nt - i;
    ++i;
  }
  ti = i;
  tj = i + r;
}

template <class DT>
__global__ __launch_bounds__(NT, 2) void gram_norm_kernel(GramArgs p) {
  constexpr int STAGE = 2 * kGramT * 128;  // A and B tiles, 64 k-values each
  __shared__ __attribute__((aligned(16))) char ring[2 * STAGE];
  __shared__ float red[NT / kWave];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int64_t item = logical_wg(blockIdx.x, gridDim.x);
  if (item >= p.items) return;
  const int64_t b = item / p.per_sample;
  int ti, tj;
  gram_item(static_cast<int>(item % p.per_sample), p.nt, ti, tj);
  const int64_t t0 = int64_t(ti) * kGramT, s0 = int64_t(tj) * kGramT;
  const uint16_t* ga = p.a + b * p.sab;
  const uint16_t* xb = p.b + b * p.sbb;
  const int nk0 = static_cast<int>(p.M / 64), nk1 = static_cast<int>(p.N / 64);
  const int nq = nk0 + nk1;

  OperandRK<4> opa, opb;  // 128 rows x 128 bytes = 16 KB = 4 KB per wave-load round
  opa.init(ga + t0 * p.lda, p.lda, p.T - t0);
  opb.init(ga + s0 * p.lda, p.lda, p.T - s0);
  FDP_LDS char* st[2] = {(FDP_LDS char*)ring, (FDP_LDS char*)ring + STAGE};
  uint32_t fa[2], fb[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    fa[i] = rk_frag_off(wm, i);
    fb[i] = rk_frag_off(wn, i) + kGramT * 128;
  }

  int iq = 0;  // next k-tile to issue (stream position)
  auto issue_next = [&](FDP_LDS char* stage) {
    const int kt = iq < nk0 ? iq : iq - nk0;
    opa.issue(stage, kt);
    opb.issue(stage + kGramT * 128, kt);
    if (++iq == nk0) {  // switch to the x rows
      opa.init(xb + t0 * p.ldb, p.ldb, p.T - t0);
      opb.init(xb + s0 * p.ldb, p.ldb, p.T - s0);
    }
  };

  f32x16 acc[2][2], gg[2][2];
  zero(acc);
  dma::wait_vm<0>();
  issue_next(st[0]);
  for (int base = 0; base < nq; base += 2) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int q = base + s;
      if (q < nq) {
        dma::wait_vm<0>();
        dma::barrier();
        if (q + 1 < nq) issue_next(st[s ^ 1]);
        const FDP_LDS char* cur = st[s];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          uint4 a[2], bb[2];
#pragma unroll
          for (int i = 0; i < 2; ++i) a[i] = read_frag_b128(cur, fa[i] ^ (ks << 5));
#pragma unroll
          for (int j = 0; j < 2; ++j) bb[j] = read_frag_b128(cur, fb[j] ^ (ks << 5));
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = dma::mfma16<DT>(a[i], bb[j], acc[i][j]);
        }
        if (q == nk0 - 1) {  // g-Gram tile complete
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) gg[i][j] = acc[i][j];
          zero(acc);
        }
      }
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) sum += gg[i][j][r] * acc[i][j][r];
  sum = wave_sum(sum);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float w = ti == tj ? 1.f : 2.f;
    p.partials[item] = w * ((red[0] + red[1]) + (red[2] + red[3]));
  }
}

// ------------------------------------------------------------ clipped sum
// Tile id -> output tile of a BM x BN geometry, banded like tile_coords().
template <class G>
__device__ __forceinline__ void tile_coords_g(const Args& p, int tile, int64_t& m0, int64_t& n0) {
  const int per_band = kBandRows * p.tiles_n;
  const int band = tile / per_band, in_band = tile % per_band;
  const int rows_left = p.tiles_m - band * kBandRows;
  const int band_rows = rows_left < kBandRows ? rows_left : kBandRows;
  m0 = int64_t(band * kBandRows + in_band % band_rows) * G::BM;
  n0 = int64_t(in_band / band_rows) * G::BN;
}

// Writes the rows of the waves in row-half h (tile rows h*WM .. h*WM+WM-1)
// through LDS as 16-byte chunks: out[m, n] = scale * acc (+ noise_scale *
// noise) in the output dtype, or fp32 rows of a group partial (ldg = N).
template <class OT, class G>
__device__ inline void store_half(const Args& p, int64_t m0, int64_t n0, int h,
                                  const f32x16 (&acc)[G::FI][G::FJ], float scale, float* lds,
                                  float* group_rows) {
  using S = typename OT::storage;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wn = (wave & 1) * G::WN;
  if ((wave >> 1) == h) {
#pragma unroll
    for (int i = 0; i < G::FI; ++i)
#pragma unroll
      for (int j = 0; j < G::FJ; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          lds[acc_row(0, i, lane, r) * G::BN + acc_col(wn, j, lane)] = acc[i][j][r] * scale;
  }
  __syncthreads();
  const int64_t mh = m0 + h * G::WM;
  if (group_rows != nullptr) {  // fp32 partial rows [M, N]
    constexpr int CPR = G::BN / 4;
    const bool vec = p.N % 4 == 0;
    for (int q = threadIdx.x; q < G::WM * CPR; q += NT) {
      const int row = q / CPR, col = (q % CPR) * 4;
      const int64_t m = mh + row, n = n0 + col;
      if (m >= p.M || n >= p.N) continue;
      const float* src = lds + row * G::BN + col;
      float* dst = group_rows + m * p.N + n;
      if (vec && n + 4 <= p.N) {
        *reinterpret_cast<float4*>(dst) = *reinterpret_cast<const float4*>(src);
      } else {
        for (int e = 0; e < 4 && n + e < p.N; ++e) dst[e] = src[e];
      }
    }
  } else {
    constexpr int E = 16 / sizeof(S);
    constexpr int CPR = G::BN / E;
    S* out = static_cast<S*>(p.out);
    const bool vec = (reinterpret_cast<uintptr_t>(out) % 16 == 0) && (p.ldo % E == 0);
    const NoiseSrc nz = p.noise.resolved();  // a value copy: no address of the kernel argument is taken
  const int zvec = noise_chunks<E>(nz, p.N);
#pragma unroll 1
    for (int q = threadIdx.x; q < G::WM * CPR; q += NT) {
      const int row = q / CPR, col = (q % CPR) * E;
      const int64_t m = mh + row, n = n0 + col;
      if (m >= p.M || n >= p.N) continue;
      const float* src = lds + row * G::BN + col;
      float v[E];
#pragma unroll
      for (int e = 0; e < E; ++e) v[e] = src[e];
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
  __syncthreads();
}

// Grid: tiles x groups workgroups (XCD-aware numbering; group-major).  Group g
// sums samples [g*spg, min(B, (g+1)*spg)) of one output tile.
// BOP 1 / 2: also the column sums and squares of operand a / b for its bias
// (bias_finish, run by bias_finish_kernel after this kernel): taken from the
// fragments of every sample, also of a sample whose clip factor is zero
// (its fragments are then read for the bias only).
// Samples per group whose clip factors the clipped-sum kernel forms itself
// (more: wgrad_factor_kernel forms them before it).
constexpr int kSumFacMax = 256;

template <class DT, class G, int S, int BOP = 0>
__global__ __launch_bounds__(NT, 2) void clipsum_kernel(Args p) {
  static_assert(S >= 2 && S <= 4, "ring depth");
  static_assert(S * G::STAGE >= G::WM * G::BN * 4, "output staging reuses the ring");
  constexpr int BW = BOP == 1 ? G::BM : G::BN;      // the tile's extent along the bias axis
  constexpr int NF = (BOP == 1 ? G::FI : G::FJ) / 2;  // bias fragments summed per wave
  static_assert(BOP == 0 || NF >= 1, "two waves share each row (column) of fragments");
  __shared__ __attribute__((aligned(16))) char ring[S * G::STAGE];
  __shared__ float bcol[BOP != 0 ? BW : 1];
  __shared__ float bred[NT / kWave];
  __shared__ float cfac[kSumFacMax];  // the group's clip factors (fac_parts > 0)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * G::WM, wn = (wave & 1) * G::WN;
  const int tiles = p.tiles_m * p.tiles_n;
  const int lw = logical_wg(blockIdx.x, gridDim.x);
  const int g = lw / tiles, tile = lw % tiles;
  int64_t m0, n0;
  tile_coords_g<G>(p, tile, m0, n0);
  const int64_t b0 = int64_t(g) * p.spg;
  const int64_t b1 = b0 + p.spg < p.B ? b0 + p.spg : p.B;
  const int nsamp = static_cast<int>(b1 - b0);
  const int nk = static_cast<int>((p.K + G::BK - 1) / G::BK);
  const int nq = nsamp * nk;
  const uint16_t* pa = static_cast<const uint16_t*>(p.a);
  const uint16_t* pb = static_cast<const uint16_t*>(p.b);
  // bias: the tile's index along the other axis; of the two waves sharing a
  // row (column) of fragments, this one sums fragments bws * NF .. + NF - 1:
  // its tile columns from bcl (bias_frag)
  const int bother = BOP == 1 ? static_cast<int>(n0 / G::BN) : static_cast<int>(m0 / G::BM);
  const int bws = BOP == 1 ? (wave & 1) : (wave >> 1);
  const int bcl = (BOP == 1 ? wm : wn) + 32 * NF * bws;
  const int blim = bias_limit(p.bias_len, BOP == 1 ? m0 : n0);
  float bcs[NF > 0 ? NF : 1] = {}, bsq = 0.f;
  (void)bother;
  (void)bws;
  (void)bcl;
  (void)blim;

  dma::FragOffsets<G> fo;
  fo.init(wm, wn);
  dma::Job<G> job;
  int iu = 0, ik = 0;
  if (nq > 0) job.init(pa + b0 * p.sab, p.lda, pb + b0 * p.sbb, p.ldb, p.K, m0, n0);
  auto issue_next = [&](FDP_LDS char* stage) {
    job.issue(stage, ik);
    if (++ik == nk) {
      ik = 0;
      if (++iu < nsamp) {
        const int64_t b = b0 + iu;
        job.retarget(pa + b * p.sab, p.lda, pb + b * p.sbb, p.ldb, p.K);
      }
    }
  };
  auto stage = [&](int s) { return (FDP_LDS char*)ring + s * G::STAGE; };

  f32x16 acc[G::FI][G::FJ];
#pragma unroll
  for (int i = 0; i < G::FI; ++i)
#pragma unroll
    for (int j = 0; j < G::FJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  float c_prev = 0.f;
  bool any = false, live = false;
  int cu = 0, ck = 0;
  int bk = 0;  // ck % bias_P (the bias counts k-tile ck when bk == bother)
  dma::wait_vm<0>();
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nq) issue_next(stage(s));
  if (p.fac_parts > 0) {
    // the clip factors of the group's samples, while the first stages load:
    // wave w takes samples w, w + 4, ... and sums each one's partials
    // lane-strided, then across the wave (the order of wgrad_factor_kernel);
    // the workgroup of tile 0 reports them.  (Waiting for these loads also
    // waits for the stages issued before them.)
    float C = p.C, clamp = p.clamp;
    if (p.clip_args_dev != nullptr) {
      C = p.clip_args_dev[0];
      clamp = p.clip_args_dev[1];
    }
    for (int j = wave; j < nsamp; j += NT / kWave) {
      const float* part = p.partials + (b0 + j) * p.fac_parts;
      float s = 0.f;
      for (int t = lane; t < p.fac_parts; t += kWave) s += part[t];
      const float n = sqrtf(wave_sum(s));
      if (lane == 0) {
        const float c = clip_factor(n, C, clamp);
        cfac[j] = c;
        if (tile == 0) {
          if (p.norms_out) p.norms_out[b0 + j] = n;
          if (p.factors_out) p.factors_out[b0 + j] = c;
        }
      }
    }
  }
  for (int base = 0; base < nq; base += S) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int q = base + s;
      if (q < nq) {
        const int ahead = nq - 1 - q;
        dma::wait_tiles<G::LOADS>(ahead < S - 2 ? ahead : S - 2);
        dma::barrier();
        if (q + S - 1 < nq) issue_next(stage((s + S - 1) % S));
        if (ck == 0) {  // sample b0 + cu starts: rescale to its factor
          const float c = p.fac_parts > 0 ? cfac[cu] : p.factors[b0 + cu];
          live = c != 0.f;  // a zero factor contributes exactly nothing
          if (live) {
            if (any) {
              const float ratio = c_prev / c;
#pragma unroll
              for (int i = 0; i < G::FI; ++i)
#pragma unroll
                for (int j = 0; j < G::FJ; ++j)
#pragma unroll
                  for (int r = 0; r < 16; ++r) acc[i][j][r] *= ratio;
            }
            c_prev = c;
            any = true;
          }
        }
        if (live) dma::compute_stage<DT, G>(stage(s), fo, acc);
        if constexpr (BOP != 0) {
          if (bk == bother)  // a counted k-tile
            bias_from_stage<DT, G, BOP, NF>(stage(s), BOP == 1 ? wm : wn, NF * bws, bcs, bsq,
                                            bcl, blim);
          bk = bk + 1 == p.bias_P ? 0 : bk + 1;
        }
        if (++ck == nk) {
          bk = 0;
          if constexpr (BOP != 0) {  // the sample's bias partials
            bias_fold<NF>(bcs, bsq, bcol, bred, bcl);
            dma::barrier();
            bias_store<BW>(p, bcol, (bred[0] + bred[1]) + (bred[2] + bred[3]), b0 + cu, tile,
                           tiles, BOP == 1 ? m0 : n0, bother);
          }
          ck = 0;
          ++cu;
        }
      }
    }
  }
  dma::barrier();  // the ring is free for the output staging

  const bool single = p.groups == 1;
  const float scale = any ? c_prev * (single ? p.out_scale : 1.f) : 0.f;
  float* lds = reinterpret_cast<float*>(ring);
  float* grows = single ? nullptr : p.group_out + int64_t(g) * p.M * p.N;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (!single) store_half<F32, G>(p, m0, n0, h, acc, scale, lds, grows);
    else if (p.out_dtype == FDP_BF16) store_half<BF16, G>(p, m0, n0, h, acc, scale, lds, nullptr);
    else if (p.out_dtype == FDP_F16) store_half<F16, G>(p, m0, n0, h, acc, scale, lds, nullptr);
    else store_half<F32, G>(p, m0, n0, h, acc, scale, lds, nullptr);
  }
}

// ------------------------------------------------------------------ host
// Geometry of the clipped-sum pass: 128 x 256 output tiles (each wave 64 x 128,
// 2 x 4 MFMA blocks), 32-deep k-tiles in a 3-stage ring (72 KB, two
// workgroups per CU).
using SumGeom = dma::Geom<128, 256, 32>;
constexpr int kSumStages = 3;

struct StreamPlan {
  int sum_tiles_m, sum_tiles_n, sum_groups, sum_spg;
  int gram_nt, gram_per_sample;
  bool gram;  // the Gram norm is used (cheaper and shape-compatible)
};

inline StreamPlan stream_plan(int64_t B, int64_t K, int64_t M, int64_t N, int cus) {
  StreamPlan s{};
  s.sum_tiles_m = static_cast<int>((M + SumGeom::BM - 1) / SumGeom::BM);
  s.sum_tiles_n = static_cast<int>((N + SumGeom::BN - 1) / SumGeom::BN);
  const int64_t tiles = int64_t(s.sum_tiles_m) * s.sum_tiles_n;
  // split the batch into groups while tiles x groups workgroups stay within
  // one wave of two per CU (a second, partial wave would cost a whole extra
  // tile time), keeping the fp32 group partials at or below B*M*N bytes
  int64_t want = 2 * int64_t(cus) / tiles;
  const int64_t cap = B / 4 > 1 ? B / 4 : 1;
  if (want > cap) want = cap;
  if (want < 1) want = 1;
  s.sum_spg = static_cast<int>((B + want - 1) / want);
  s.sum_groups = static_cast<int>((B + s.sum_spg - 1) / s.sum_spg);
  s.gram_nt = static_cast<int>((K + kGramT - 1) / kGramT);
  s.gram_per_sample = s.gram_nt * (s.gram_nt + 1) / 2;
  const double direct = double(K) * M * N;
  const double gram = double(s.gram_per_sample) * kGramT * kGramT * double(M + N);
  s.gram = M % 64 == 0 && N % 64 == 0 && K > 0 && gram < direct;
  return s;
}

template <class DT>
hipError_t launch_gram_norm(const GramArgs& g, hipStream_t s) {
  if (g.items <= 0) return hipSuccess;
  hipLaunchKernelGGL(gram_norm_kernel<DT>, dim3(static_cast<unsigned>(g.items)), dim3(NT), 0, s, g);
  return hipGetLastError();
}

// Partials per bias output of the clipped-sum pass (tiles along the other axis).
inline int stream_bias_P(const StreamPlan& sp, int bias_op) {
  return bias_op == 1 ? sp.sum_tiles_n : sp.sum_tiles_m;
}

// The clipped-sum pass; with a.bias_op, also the bias (bias_finish_kernel
// after the pass, one workgroup per kBiasCols outputs).
template <class DT>
hipError_t launch_clipsum(Args a, const StreamPlan& sp, hipStream_t s) {
  a.tiles_m = sp.sum_tiles_m;
  a.tiles_n = sp.sum_tiles_n;
  a.groups = sp.sum_groups;
  a.spg = sp.sum_spg;
  const int tiles = a.tiles_m * a.tiles_n;
  const unsigned grid = static_cast<unsigned>(tiles * a.groups);
  if (a.bias_op == 0) {
    hipLaunchKernelGGL((clipsum_kernel<DT, SumGeom, kSumStages, 0>), dim3(grid), dim3(NT), 0, s, a);
    return hipGetLastError();
  }
  a.bias_P = stream_bias_P(sp, a.bias_op);
  if (a.bias_op == 1)
    hipLaunchKernelGGL((clipsum_kernel<DT, SumGeom, kSumStages, 1>), dim3(grid), dim3(NT), 0, s, a);
  else
    hipLaunchKernelGGL((clipsum_kernel<DT, SumGeom, kSumStages, 2>), dim3(grid), dim3(NT), 0, s, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  int64_t nfin = (a.bias_len + kBiasCols - 1) / kBiasCols;
  if (nfin > 2048) nfin = 2048;
  hipLaunchKernelGGL(bias_finish_kernel<0>, dim3(static_cast<unsigned>(nfin)), dim3(NT), 0, s, a,
                     tiles);
  return hipGetLastError();
}

// Per-dtype instantiations (wgrad_stream_{bf16,f16}.hip).
hipError_t launch_gram_norm_bf16(const GramArgs& g, hipStream_t s);
hipError_t launch_gram_norm_f16(const GramArgs& g, hipStream_t s);
hipError_t launch_clipsum_bf16(const Args& a, const StreamPlan& sp, hipStream_t s);
hipError_t launch_clipsum_f16(const Args& a, const StreamPlan& sp, hipStream_t s);

}  // namespace wg
}  // namespace fdp
