// Input gradient of a DP Linear / Conv1D layer on CDNA4 MFMA (gfx950):
//
//   dX[m, n] = sum_k g[m, k] W(k, n),   g = grad_output [M = B*T, K = out]
//
// with W(k, n) = W[k, n] for a Linear weight [out, in] (FDP_DGRAD_NN) or
// W[n, k] for a Conv1D weight [in, out] (FDP_DGRAD_NT).  This is the unclipped
// third product of the layer's backward (flashdp/layers/linear.py:62-67 forms
// it with torch's matmul); the clipped weight gradient reads the same g.
//
// The core is the LDS-DMA / ds_read MFMA core of the clipped products
// (gemm_dma.hpp): 8 waves of 64 x (BN / 2) outputs each, a 2-stage ring of
// 64-deep k-tiles (a 3-stage ring of 32-deep ones, with half the MFMAs
// between two workgroup barriers, took 57-61 against 53.6-54.4 us at the
// cfg2 and cfg3 shapes).  g has k contiguous, so its tiles are kept in LDS as rows
// of 64 k-values and read with plain ds_read_b128 (Geom::AKC); a Linear weight
// is k-strided (the clipped products' transposing reads), a Conv1D weight
// k-contiguous (Geom::BKC).
//
// Work map: one workgroup per output tile of 256 or 128 rows of g by 192
// columns of dX (the host picks the height that needs the fewer rounds of
// workgroups over the CUs: cfg2's 8192 x 768 outputs are 128 tiles of 256
// rows but 256 of 128), XCD-contiguous.  No workgroup waits for another.
#pragma once

#include "gemm_dma.hpp"

namespace fdp {
namespace dg {

constexpr int kThreads = 512;
constexpr int kBK = 64;     // k-tile depth
constexpr int kStages = 2;  // ring stages (64 KB each)
constexpr int kBM = 256, kBN = 192;  // output tile: 256 rows of g x 192 columns of dX
constexpr int kBMHalf = 128;         // or 128 rows (32 per wave), when 256 leave CUs idle
constexpr int kXcds = 8;

struct DgradArgs {
  const uint16_t* g;  // [M, K], row stride ldg
  const uint16_t* w;  // NN: [K, N] row stride ldw; NT: [N, K] row stride ldw
  uint16_t* out;      // [M, N], row stride ldo (g's dtype)
  int vec_out;        // out rows are 16-byte aligned (ldo % 8 == 0, out 16-byte aligned)
  int64_t M, N, K;
  int64_t ldg, ldw, ldo;
  int tiles_m, tiles_n;
  int nk;             // 64-deep k-tiles of the contraction
};

// Hardware workgroup -> logical item, XCD-contiguous: workgroups are dealt
// round-robin to the 8 XCDs, so item ranges [x * n / 8, (x + 1) * n / 8) run
// on XCD x and neighbouring items (the n-tiles of one row band of g) share
// that XCD's L2.
__device__ __forceinline__ int item_of(int hw, int n) {
  if (n % kXcds != 0) return hw;
  return (hw % kXcds) * (n / kXcds) + hw / kXcds;
}

template <class G, bool WKC>
struct DJob {
  dma::Operand<G::LOADS_A, G::BK> a;
  dma::Operand<G::LOADS_B, G::BK> b;
  // output tile (m0, n0)
  __device__ __forceinline__ void init(const DgradArgs& p, int64_t m0, int64_t n0) {
    a.template init_kc<G::BM>(p.g, p.ldg, p.M, m0);
    if constexpr (WKC) b.template init_kc<G::BN>(p.w, p.ldw, p.N, n0);
    else b.template init<G::BN>(p.w, p.ldw, p.K, n0);
  }
  __device__ __forceinline__ void issue(FDP_LDS char* stage, int kt) const {
    a.issue(stage, kt);
    b.issue(stage + G::TILE_A, kt);
  }
};

template <class DT, int BM, int BN, bool WKC>
__global__ __launch_bounds__(kThreads, 1) void dgrad_kernel(DgradArgs p) {
  using G = dma::Geom<BM, BN, kBK, 4, 2, true, WKC>;
  static_assert(G::NW == 8, "8 waves: 4 along g's rows, 2 along dX's columns");
  constexpr int WMR = G::WM;  // rows of g per wave (BM / 4)
  constexpr int FI = G::FI, FJ = G::FJ;
  __shared__ __attribute__((aligned(16))) char st0[G::STAGE];
  __shared__ __attribute__((aligned(16))) char st1[G::STAGE];
  static_assert(kStages == 2, "two ring stages");
  const dma::Stages stages{{(FDP_LDS char*)(st0), (FDP_LDS char*)(st1), (FDP_LDS char*)(st0),
                            (FDP_LDS char*)(st1)}};
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * WMR, wn = (wave & 1) * (BN / 2);

  const int tile = item_of(blockIdx.x, p.tiles_m * p.tiles_n);
  const int64_t m0 = int64_t(tile / p.tiles_n) * BM, n0 = int64_t(tile % p.tiles_n) * BN;

  f32x16 acc[FI][FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  {
    dma::FragOffsets<G> fo;
    fo.init(wm, wn);
    DJob<G, WKC> job;
    job.init(p, m0, n0);
    dma::gemm_pipe<DT, G, kStages>(job, p.nk, fo, stages, acc);
  }

  // ---- store dX in g's dtype.  Each wave stages its WMR x (BN/2) sub-tile
  // in LDS (rows of kStageRow bytes, so that the two rows one store
  // instruction writes, 4 apart, fall on different banks) and writes it back
  // as 16-byte row segments.  The ring is free (gemm_pipe ended on a
  // barrier): four sub-tiles per ring stage.
  constexpr int WN = BN / 2, CH = WN / 8;  // columns, 16-byte chunks per sub-tile row
  constexpr int kStageRow = WN * 2 + 16;
  constexpr int kPerStage = G::STAGE / (WMR * kStageRow);  // sub-tiles a ring stage holds
  static_assert(kPerStage * kStages >= 8, "every wave's sub-tile fits the ring at once");
  static_assert(WMR * CH % 64 == 0, "whole rounds of 16-byte chunks per wave");
  FDP_LDS char* const sub = stages.get(wave / kPerStage) + (wave % kPerStage) * WMR * kStageRow;
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        *reinterpret_cast<FDP_LDS uint16_t*>(sub + row * kStageRow + (32 * j + (lane & 31)) * 2) =
            DT::from_f32(acc[i][j][r]);
      }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's writes, read below
#pragma unroll
  for (int k = 0; k < WMR * CH / 64; ++k) {
    const int c = lane + 64 * k, row = c / CH, ch = c % CH;
    const u32x4 v = *reinterpret_cast<const FDP_LDS u32x4*>(sub + row * kStageRow + ch * 16);
    const int64_t grow = m0 + wm + row, gcol = n0 + wn + ch * 8;
    if (grow >= p.M) continue;
    uint16_t* dst = p.out + grow * p.ldo + gcol;
    if (p.vec_out && gcol + 8 <= p.N) {
      *reinterpret_cast<uint4*>(dst) = make_uint4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (gcol + e < p.N) dst[e] = static_cast<uint16_t>(v[e >> 1] >> (16 * (e & 1)));
    }
  }
}

// Instantiated per dtype in dgrad_{bf16,f16}.hip.  (A 256-wide tile needs
// 128 accumulators per thread and spills beside the double-buffered fragments
// at two waves per SIMD; 192 columns keep 96 and about 200 VGPRs.)
template <class DT>
hipError_t launch_dgrad_t(const DgradArgs& a, int bm, bool wkc, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(a.tiles_m * a.tiles_n)), block(kThreads);
  if (bm == kBM) {
    if (wkc) hipLaunchKernelGGL((dgrad_kernel<DT, kBM, kBN, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((dgrad_kernel<DT, kBM, kBN, false>), grid, block, 0, s, a);
  } else {
    if (wkc) hipLaunchKernelGGL((dgrad_kernel<DT, kBMHalf, kBN, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((dgrad_kernel<DT, kBMHalf, kBN, false>), grid, block, 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_dgrad_bf16(const DgradArgs& a, int bm, bool wkc, hipStream_t s);
hipError_t launch_dgrad_f16(const DgradArgs& a, int bm, bool wkc, hipStream_t s);

}  // namespace dg
}  // namespace fdp
