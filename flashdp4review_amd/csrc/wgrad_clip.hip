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
// Three schedules, chosen per call:
//   single pass (wgrad_core.hpp): 16-bit TN operands whose 128x128 output tiles
//     fit the co-resident grid: every per-sample tile product stays in the
//     register file across one grid barrier.
//   streamed two-pass (wgrad_stream.hpp): the other 16-bit TN problems with
//     aligned rows (layers larger than the resident grid): Gram-form or direct
//     per-sample norms, then one clipped-sum contraction per output tile.
//   generic two-pass (below): fp32 inputs, NN layout, unaligned rows --
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
// Generic tiles: 128x128 outputs per 256-thread workgroup (4 waves, 64x64 each as 2x2
// blocks of 32x32 MFMA).  16-bit inputs use v_mfma_f32_32x32x16_{bf16,f16} with
// BK=64; fp32 inputs use v_mfma_f32_32x32x2_f32 with BK=16.  Global loads are
// 16-byte and coalesced along the contiguous dimension; for operands whose
// contraction axis is strided (every TN operand) the 16-bit loader transposes
// 4x8 element blocks in registers (v_perm_b32) so that each MFMA lane then reads
// its 8 consecutive k-values with one ds_read_b128.  LDS rows are XOR-swizzled
// in 16-byte chunks to spread both the transposing writes and the fragment
// reads over the banks.  LDS is double-buffered: the next k-tile's global loads
// are issued before the current tile's MFMAs.
#include <cstdlib>

#include "wgrad_stream.hpp"
#include <tuple>

#include "wgrad_wide.hpp"

namespace fdp {
namespace wg {

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
// One wavefront per sample: ||G_b|| = sqrt(sum over tiles of partials[b, :]),
// summed in a fixed lane/stride order; c_b = min(clamp, C/(||G_b|| + 1e-10)).
__global__ __launch_bounds__(NT) void wgrad_factor_kernel(const float* partials, int64_t B,
                                                           int tiles, float C, float clamp,
                                                           const float* clip_args_dev,
                                                           int noclip, float* fac_ws,
                                                           float* norms, float* factors,
                                                           int* err) {
  (void)err;  // the two-pass schedule has no bounded waits: the status word stays as it is
  if (clip_args_dev != nullptr) {
    C = clip_args_dev[0];
    clamp = clip_args_dev[1];
  }
  const int lane = threadIdx.x & 63;
  const int64_t waves = int64_t(gridDim.x) * (NT / kWave);
  for (int64_t b = int64_t(blockIdx.x) * (NT / kWave) + (threadIdx.x >> 6); b < B; b += waves) {
    float n = 0.f;
    if (!noclip) {
      float s = 0.f;
      for (int t = lane; t < tiles; t += kWave) s += partials[b * tiles + t];
      n = sqrtf(wave_sum(s));
    }
    if (lane == 0) {
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
  const NoiseSrc nz = p.noise.resolved();
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
          if (nz.on()) v += p.noise_scale * nz.at(m * p.N + n);
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
  const NoiseSrc nz = p.noise.resolved();
  for (int64_t e = int64_t(blockIdx.x) * NT + threadIdx.x; e < MN; e += int64_t(gridDim.x) * NT) {
    float s = 0.f;
    for (int g = 0; g < p.groups; ++g) s += p.group_out[int64_t(g) * MN + e];
    float v = s * p.out_scale;
    if (nz.on()) v += p.noise_scale * nz.at(e);
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


// Workspace layout (both schedules):
//   [0, 256)            status word (int), barrier and finished-workgroup
//                       counters (uint); zero between calls, except a status set
//                       by an expired wait (the only words a reused workspace
//                       must carry over: everything after them is rewritten)
//   off_turn            per-tile counters [tiles] (uint)
//   off_partials        partials [B, max(tiles, Gram items per sample)] (fp32)
//   two-pass:  off_factors [B], off_group [groups, M, N] (fp32)
//   one-pass:  off_slots [groups, tiles, BM*BN] (fp32) per-group tile sums,
//              off_chunk [M, N] (fp32) running sum when the batch needs
//              more than one launch
struct Plan {
  int tiles_m, tiles_n, tiles;
  int spg, groups;
  StreamPlan sp;  // streamed two-pass schedule (16-bit TN operands)
  WidePlan wp;    // wide single-pass schedule (wp.wgm == 0: not used)
  size_t off_turn, off_partials, off_factors, off_group, off_slots, off_chunk;
  size_t off_wide_partials, off_wide_slots, off_wide_bias_part, off_wide_bias_sq;
  size_t total_two_pass, total_fused, total_wide, total;
};

// Smallest share of the CUs the wide kernel's products must fill by default.
constexpr double kWideMinFill = 0.7;

// Polls before a grid wait of the single-pass kernel gives up (seconds of
// waiting).  FDP_WGRAD_SPIN_LIMIT overrides it so that tests can exercise the
// expiry path with every kernel still running to completion.
unsigned spin_limit() {
  const char* e = getenv("FDP_WGRAD_SPIN_LIMIT");
  if (e != nullptr && *e != '\0') return static_cast<unsigned>(strtoul(e, nullptr, 10));
  return kSpinLimit;
}

int num_cus() { return host::device_cus(); }

// lda/ldb: the row strides the call will use (the size query assumes
// contiguous operands, lda = M and ldb = N, which the layers pass).
Plan make_plan(int64_t B, int64_t K, int64_t M, int64_t N, int cus, int flags, int64_t lda = 0,
               int64_t ldb = 0) {
  Plan pl{};
  pl.tiles_m = static_cast<int>((M + BM - 1) / BM);
  pl.tiles_n = static_cast<int>((N + BN - 1) / BN);
  pl.tiles = pl.tiles_m * pl.tiles_n;
  // Two-pass clipped sum: split the batch into groups until there are ~2
  // workgroups per CU, keeping the fp32 group partials (groups*M*N*4 bytes) at
  // or below B*M*N bytes.
  int64_t want = (2 * int64_t(cus) + pl.tiles - 1) / pl.tiles;
  const int64_t cap = B / 4 > 1 ? B / 4 : 1;
  if (want > cap) want = cap;
  if (want < 1) want = 1;
  pl.spg = static_cast<int>((B + want - 1) / want);
  pl.groups = static_cast<int>((B + pl.spg - 1) / pl.spg);
  pl.sp = stream_plan(B, K, M, N, cus);
  pl.off_turn = kWsHead;
  pl.off_partials = pl.off_turn + align_up(sizeof(unsigned) * size_t(pl.tiles));
  const size_t per_sample =
      size_t(pl.tiles > pl.sp.gram_per_sample ? pl.tiles : pl.sp.gram_per_sample);
  const size_t after_partials = pl.off_partials + align_up(sizeof(float) * size_t(B) * per_sample);
  pl.off_factors = after_partials;
  pl.off_group = pl.off_factors + align_up(sizeof(float) * size_t(B));
  const int max_groups = pl.groups > pl.sp.sum_groups ? pl.groups : pl.sp.sum_groups;
  pl.total_two_pass =
      pl.off_group + (max_groups > 1 ? align_up(sizeof(float) * size_t(max_groups) * M * N) : 0);
  const GroupPlan gp = group_plan(B, pl.tiles, 2 * cus);
  pl.off_slots = after_partials;
  pl.off_chunk = pl.off_slots;
  pl.total_fused = 0;
  if (gp.chunk > 0) {
    pl.off_chunk += align_up(sizeof(uint16_t) * size_t(gp.max_nwg) * BM * BN);
    pl.total_fused = pl.off_chunk + (gp.chunk < B ? sizeof(float) * size_t(M) * N : 0);
  }
  pl.total = pl.total_two_pass > pl.total_fused ? pl.total_two_pass : pl.total_fused;
  if ((flags & FDP_WGRAD_NARROW) == 0 && K > 0) {
    pl.wp = wide_plan(B, K, M, N, lda > 0 ? lda : M, ldb > 0 ? ldb : N, cus,
                      (flags & FDP_WGRAD_WIDE) ? 0.0 : kWideMinFill);
    if (flags & FDP_WGRAD_UNPAIRED) pl.wp.pair = 0;
    if (pl.wp.any()) {
      pl.off_wide_partials = kWsHead;
      pl.off_wide_slots = pl.off_wide_partials + align_up(pl.wp.partial_bytes);
      pl.off_wide_bias_part = pl.off_wide_slots + align_up(pl.wp.slot_bytes);
      pl.off_wide_bias_sq = pl.off_wide_bias_part + align_up(pl.wp.bias_part_bytes);
      pl.total_wide = pl.off_wide_bias_sq + pl.wp.bias_sq_bytes;
      if (pl.total_wide > pl.total) pl.total = pl.total_wide;
    }
  }
  return pl;
}

bool valid_dtype(int d) { return d == FDP_F32 || d == FDP_F16 || d == FDP_BF16; }

// make_plan depends only on its arguments: computed once per shape.
Plan cached_plan(int64_t B, int64_t K, int64_t M, int64_t N, int cus, int flags, int64_t lda = 0,
                 int64_t ldb = 0) {
  using Key = std::tuple<int64_t, int64_t, int64_t, int64_t, int, int, int64_t, int64_t>;
  static host::ShapeCache<Key, Plan> cache;
  return cache.get(Key{B, K, M, N, cus, flags, lda, ldb},
                   [&] { return make_plan(B, K, M, N, cus, flags, lda, ldb); });
}

template <class Core, int LAYOUT, bool VEC>
hipError_t launch_passes(const Args& a, const Plan& pl, bool noclip, float C, float clamp,
                         const float* clip_args_dev, float* norms, float* factors, float* fac_ws,
                         hipStream_t s) {
  const dim3 block(NT);
  if (!noclip) {
    hipLaunchKernelGGL((wgrad_norm_kernel<Core, LAYOUT, VEC>), dim3(pl.tiles, a.B), block,
                       Core::SMEM, s, a);
  }
  const unsigned fb = static_cast<unsigned>((a.B + (NT / kWave) - 1) / (NT / kWave));
  hipLaunchKernelGGL(wgrad_factor_kernel, dim3(fb < 1024 ? fb : 1024), block, 0, s, a.partials,
                     a.B, pl.tiles, C, clamp, clip_args_dev, noclip ? 1 : 0, fac_ws, norms,
                     factors, a.err);
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

// Streamed two-pass schedule for 16-bit TN operands with aligned rows: Gram
// (or direct) norms, factors, then one clipped-sum contraction per output tile.
template <class DT>
hipError_t launch_stream(Args a, const Plan& pl, bool noclip, float C, float clamp,
                         const float* clip_args_dev, float* norms, float* factors, float* fac_ws,
                         hipStream_t s) {
  const dim3 block(NT);
  int per_sample = pl.tiles;
  if (!noclip) {
    if (pl.sp.gram) {
      GramArgs g{};
      g.a = static_cast<const uint16_t*>(a.a);
      g.b = static_cast<const uint16_t*>(a.b);
      g.B = a.B;
      g.T = a.K;
      g.M = a.M;
      g.N = a.N;
      g.sab = a.sab;
      g.lda = a.lda;
      g.sbb = a.sbb;
      g.ldb = a.ldb;
      g.nt = pl.sp.gram_nt;
      g.per_sample = pl.sp.gram_per_sample;
      g.items = a.B * g.per_sample;
      g.partials = a.partials;
      per_sample = g.per_sample;
      const hipError_t e = DT::code == FDP_BF16 ? launch_gram_norm_bf16(g, s) : launch_gram_norm_f16(g, s);
      if (e != hipSuccess) return e;
    } else {
      hipLaunchKernelGGL((wgrad_norm_kernel<Core16<DT>, FDP_LAYOUT_TN, true>), dim3(pl.tiles, a.B),
                         block, Core16<DT>::SMEM, s, a);
    }
  }
  // The clipped-sum kernel forms the factors from the partials itself (saving
  // a launch between the passes) unless the call has no clipping or its
  // sample groups are larger than it stages.
  a.fac_parts = 0;
  if (!noclip && pl.sp.sum_spg <= kSumFacMax) {
    a.fac_parts = per_sample;
    a.C = C;
    a.clamp = clamp;
    a.clip_args_dev = clip_args_dev;
    a.norms_out = norms;
    a.factors_out = factors;
  } else {
    const unsigned fb = static_cast<unsigned>((a.B + (NT / kWave) - 1) / (NT / kWave));
    hipLaunchKernelGGL(wgrad_factor_kernel, dim3(fb < 1024 ? fb : 1024), block, 0, s, a.partials,
                       a.B, per_sample, C, clamp, clip_args_dev, noclip ? 1 : 0, fac_ws, norms,
                       factors, a.err);
  }
  const hipError_t e = DT::code == FDP_BF16 ? launch_clipsum_bf16(a, pl.sp, s) : launch_clipsum_f16(a, pl.sp, s);
  if (e != hipSuccess) return e;
  if (pl.sp.sum_groups > 1) {
    a.groups = pl.sp.sum_groups;
    const int64_t MN = a.M * a.N;
    int64_t nb = (MN + NT - 1) / NT;
    if (nb > 4096) nb = 4096;
    hipLaunchKernelGGL(wgrad_finalize_kernel, dim3(static_cast<unsigned>(nb)), block, 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace

extern "C" int fdp_wgrad_clip_workspace_size(int64_t B, int64_t K, int64_t M, int64_t N,
                                             int dtype, int flags, size_t* bytes) {
  (void)flags;
  if (bytes == nullptr) return FDP_ERR_ARG;
  if (!valid_dtype(dtype)) return FDP_ERR_DTYPE;
  if (B < 1 || M < 1 || N < 1 || K < 0) return FDP_ERR_SHAPE;
  *bytes = cached_plan(B, K, M, N, num_cus(), flags).total;
  return FDP_OK;
}

int fdp::wgrad_check_args(const void* a, const void* b, int64_t B, int64_t K, int64_t M,
                          int64_t N, int64_t lda, int64_t ldb, int layout, int dtype,
                          const void* out, int64_t ldo, int out_dtype, const float* norms,
                          int flags) {
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) return FDP_ERR_DTYPE;
  if (layout != FDP_LAYOUT_TN && layout != FDP_LAYOUT_NN) return FDP_ERR_ARG;
  if (B < 1 || M < 1 || N < 1 || K < 0) return FDP_ERR_SHAPE;
  if (ldo < N) return FDP_ERR_SHAPE;
  if (layout == FDP_LAYOUT_TN && (lda < M || ldb < N)) return FDP_ERR_SHAPE;
  if (layout == FDP_LAYOUT_NN && (lda < K || ldb < N)) return FDP_ERR_SHAPE;
  if (M * N > (int64_t(1) << 40) || B > (int64_t(1) << 31)) return FDP_ERR_SHAPE;
  if ((K > 0 && (a == nullptr || b == nullptr)) || out == nullptr) return FDP_ERR_ARG;
  if ((flags & ~(FDP_WGRAD_NOCLIP | FDP_WGRAD_TWO_PASS | FDP_WGRAD_PLAIN_LAUNCH |
                 FDP_WGRAD_CLEAN_WORKSPACE | FDP_WGRAD_WIDE | FDP_WGRAD_NARROW |
                 FDP_WGRAD_UNPAIRED)) != 0)
    return FDP_ERR_ARG;  // (FDP_WGRAD_BIAS_OF_B only with fdp_wgrad_bias_clip)
  if ((flags & FDP_WGRAD_WIDE) && (flags & FDP_WGRAD_NARROW)) return FDP_ERR_ARG;
  if ((flags & FDP_WGRAD_NOCLIP) != 0 && norms != nullptr) return FDP_ERR_ARG;
  return FDP_OK;
}

namespace {

// fdp_wgrad_clip; with `bias`, the 16-bit TN kernels (wide, grouped and
// streamed) also form the bias of operand a (bias_op 1) or b (bias_op 2) from
// the fragments they hold, with its partials in bias_part / bias_sq
// (*bias_done = true); the generic two-pass schedule leaves it to the caller.
int wgrad_clip_impl(const void* a, const void* b, int64_t B, int64_t K, int64_t M, int64_t N,
                    int64_t stride_ab, int64_t lda, int64_t stride_bb, int64_t ldb, int layout,
                    int dtype, float C, float clamp, const float* clip_args_dev, float out_scale,
                    const void* noise, float noise_scale, const fdp_noise_key* noise_key,
                    void* out, int64_t ldo, int out_dtype, float* norms, float* factors,
                    int flags, void* workspace, size_t workspace_bytes, void* stream,
                    const fdp_bias_out* bias, int bias_op, float* bias_part, float* bias_sq,
                    bool* bias_done) {
  const int bad = fdp::wgrad_check_args(a, b, B, K, M, N, lda, ldb, layout, dtype, out, ldo,
                                        out_dtype, norms, flags);
  if (bad != FDP_OK) return bad;
  const bool noclip = (flags & FDP_WGRAD_NOCLIP) != 0;

  const int cus = num_cus();
  // the workspace was sized for contiguous operands: the wide plan for the
  // actual strides is taken only if it fits that size
  const Plan pl0 = cached_plan(B, K, M, N, cus, flags);
  if (workspace == nullptr || workspace_bytes < pl0.total) return FDP_ERR_WORKSPACE;
  Plan pl = cached_plan(B, K, M, N, cus, flags, lda, ldb);
  if (pl.total > workspace_bytes) pl.wp.wgm = pl.wp.pair = 0;
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
  args.noise = make_noise(noise, out_dtype, noise_scale != 0.f ? noise_key : nullptr, 0);
  args.noise_scale = noise_scale;
  args.units = int64_t(pl.tiles) * B;
  args.err = reinterpret_cast<int*>(ws);
  args.bar = reinterpret_cast<unsigned*>(ws) + 1;
  args.epoch = reinterpret_cast<unsigned*>(ws) + 2;
  args.poison = reinterpret_cast<unsigned*>(ws) + 3;
  args.pair_flag = reinterpret_cast<unsigned*>(ws) + kPairFlag0;
  args.spin_limit = spin_limit();
  args.tile_turn = reinterpret_cast<unsigned*>(ws + pl.off_turn);
  args.tile_acc = reinterpret_cast<float*>(ws + pl.off_slots);
  args.chunk_acc = reinterpret_cast<float*>(ws + pl.off_chunk);
  args.C = C;
  args.clamp = clamp;
  args.clip_args_dev = clip_args_dev;
  args.norms_out = norms;
  args.factors_out = factors;
  if (bias != nullptr) {
    args.bias_op = bias_op;
    args.bias_P = bias_op == 1 ? pl.tiles_n : pl.tiles_m;  // the grouped kernel's tiles
    args.bias_len = bias_op == 1 ? M : N;
    args.bias_part = bias_part;
    args.bias_sq = bias_sq;
    args.bias_out = bias->out;
    args.bias_dtype = bias->out_dtype;
    args.bias_scale = bias->out_scale;
    args.bias_noise = make_noise(bias->noise, bias->out_dtype,
                                 bias->noise_scale != 0.f ? bias->noise_key : nullptr, 0);
    args.bias_noise_scale = bias->noise_scale;
    args.bias_norms = bias->norms;
    args.bias_factors = bias->factors;
  }

  // 16-byte vector loads need 16-byte aligned rows of every sample.
  const int esz = dtype == FDP_F32 ? 4 : 2;
  const int64_t vel = 16 / esz;
  const bool vec = (reinterpret_cast<uintptr_t>(a) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(b) % 16 == 0) && lda % vel == 0 &&
                   ldb % vel == 0 && stride_ab % vel == 0 && stride_bb % vel == 0;

  hipStream_t s = static_cast<hipStream_t>(stream);
  // Wide single pass: 16-bit TN inputs, aligned rows, two samples' products
  // per CU (paired) or one.
  const bool pair = pl.wp.pair != 0 && pair_records_fit(K, lda, stride_ab) &&
                    pair_records_fit(K, ldb, stride_bb);
  if (!noclip && (flags & FDP_WGRAD_TWO_PASS) == 0 && layout == FDP_LAYOUT_TN && vec && K > 0 &&
      dtype != FDP_F32 && (pair || pl.wp.wgm != 0)) {
    WideArgs w{};
    w.a = static_cast<const uint16_t*>(a);
    w.b = static_cast<const uint16_t*>(b);
    w.B = B;
    w.K = K;
    w.M = M;
    w.N = N;
    w.sab = stride_ab;
    w.lda = lda;
    w.sbb = stride_bb;
    w.ldb = ldb;
    w.tiles_m = pair ? pl.wp.pair_tiles_m : pl.wp.tiles_m;
    w.tiles_n = pair ? pl.wp.pair_tiles_n : pl.wp.tiles_n;
    w.tiles = pair ? pl.wp.pair_tiles : pl.wp.tiles;
    w.nwg = pair ? pl.wp.pair_nwg : pl.wp.nwg;
    w.partials = reinterpret_cast<float*>(ws + pl.off_wide_partials);
    w.slots = ws + pl.off_wide_slots;
    w.slot_blocks = pair ? pl.wp.pair_slot_blocks : pl.wp.slot_blocks;
    w.group_cnt = reinterpret_cast<unsigned*>(ws) + kGroupWord0;
    w.tagged = reinterpret_cast<uint64_t*>(ws + pl.off_wide_partials);
    w.out = out;
    w.ldo = ldo;
    w.out_dtype = out_dtype;
    w.out_scale = out_scale;
    w.noise = args.noise;
    w.noise_scale = noise_scale;
    w.bar = args.bar;
    w.epoch = args.epoch;
    w.poison = args.poison;
    w.err = args.err;
    w.spin_limit = args.spin_limit;
    w.C = C;
    w.clamp = clamp;
    w.clip_args_dev = clip_args_dev;
    w.norms_out = norms;
    w.factors_out = factors;
    if (bias != nullptr) {
      w.bias_op = bias_op;
      w.bias_part = reinterpret_cast<float*>(ws + pl.off_wide_bias_part);
      w.bias_sq = reinterpret_cast<float*>(ws + pl.off_wide_bias_sq);
      w.bias_tagged = reinterpret_cast<uint64_t*>(ws + pl.off_wide_bias_part);
      w.bias_sq_tagged = reinterpret_cast<uint64_t*>(ws + pl.off_wide_bias_sq);
      w.bias_out = bias->out;
      w.bias_dtype = bias->out_dtype;
      w.bias_scale = bias->out_scale;
      w.bias_noise = make_noise(bias->noise, bias->out_dtype,
                                bias->noise_scale != 0.f ? bias->noise_key : nullptr, 0);
      w.bias_noise_scale = bias->noise_scale;
      w.bias_norms = bias->norms;
      w.bias_factors = bias->factors;
    }
    {
      const int oes = out_dtype == FDP_F32 ? 4 : 2;
      w.vec_out = (reinterpret_cast<uintptr_t>(out) % (4 * oes) == 0 && ldo % 4 == 0) ? 1 : 0;
    }
    const bool plain = (flags & FDP_WGRAD_PLAIN_LAUNCH) != 0;
    if ((flags & FDP_WGRAD_CLEAN_WORKSPACE) == 0) {
      const int64_t words = int64_t(kWsHead / sizeof(unsigned));
      hipLaunchKernelGGL(clear_words_kernel<0>, dim3(static_cast<unsigned>((words + NT - 1) / NT)),
                         dim3(NT), 0, s, reinterpret_cast<unsigned*>(ws), words);
    }
    const int wgm = pair ? 1 : pl.wp.wgm;
    const hipError_t e = dtype == FDP_BF16 ? launch_wide_bf16(w, wgm, plain, s)
                                           : launch_wide_f16(w, wgm, plain, s);
    if (e == hipSuccess) {
      if (bias_done != nullptr) *bias_done = bias != nullptr;
      return FDP_OK;
    }
    if (e != hipErrorNotSupported && e != hipErrorCooperativeLaunchTooLarge) {
      (void)hipGetLastError();
      return FDP_ERR_HIP;
    }
    (void)hipGetLastError();
  }
  // Single pass: 16-bit inputs, TN layout, aligned rows, a clip to compute, K > 0.
  if (!noclip && (flags & FDP_WGRAD_TWO_PASS) == 0 && layout == FDP_LAYOUT_TN && vec && K > 0 &&
      dtype != FDP_F32 && pl.total_fused > 0) {
    const bool plain = (flags & FDP_WGRAD_PLAIN_LAUNCH) != 0;
    const bool clean = (flags & FDP_WGRAD_CLEAN_WORKSPACE) != 0;
    hipError_t e;
    if (bias != nullptr)
      e = dtype == FDP_BF16 ? launch_grouped_bias_bf16(args, cus, plain, clean, s)
                            : launch_grouped_bias_f16(args, cus, plain, clean, s);
    else
      e = dtype == FDP_BF16 ? launch_grouped_bf16(args, cus, plain, clean, s)
                            : launch_grouped_f16(args, cus, plain, clean, s);
    if (e == hipSuccess) {
      if (bias_done != nullptr) *bias_done = bias != nullptr;
      return FDP_OK;
    }
    if (e != hipErrorNotSupported && e != hipErrorCooperativeLaunchTooLarge) {
      (void)hipGetLastError();
      return FDP_ERR_HIP;
    }
    (void)hipGetLastError();
  }

  hipError_t e;
  // the streamed kernels address a sample's operands through 32-bit buffer
  // records; larger samples take the generic schedule (64-bit addressing)
  if (layout == FDP_LAYOUT_TN && vec && dtype != FDP_F32 && K > 0 && fits_record(K, lda) &&
      fits_record(K, ldb)) {
    args.group_out = pl.sp.sum_groups > 1 ? reinterpret_cast<float*>(ws + pl.off_group) : nullptr;
    e = dtype == FDP_BF16 ? launch_stream<BF16>(args, pl, noclip, C, clamp, clip_args_dev, norms,
                                                factors, fac_ws, s)
                          : launch_stream<F16>(args, pl, noclip, C, clamp, clip_args_dev, norms,
                                               factors, fac_ws, s);
    if (e != hipSuccess) return FDP_ERR_HIP;
    if (bias_done != nullptr) *bias_done = bias != nullptr;
    return FDP_OK;
  }
  args.bias_op = 0;  // the generic schedule: the caller forms the bias
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

}  // namespace

extern "C" int fdp_wgrad_clip(const void* a, const void* b, int64_t B, int64_t K, int64_t M,
                              int64_t N, int64_t stride_ab, int64_t lda, int64_t stride_bb,
                              int64_t ldb, int layout, int dtype, float C, float clamp,
                              const float* clip_args_dev, float out_scale, const void* noise,
                              float noise_scale, const fdp_noise_key* noise_key, void* out,
                              int64_t ldo, int out_dtype,
                              float* norms, float* factors, int flags, void* workspace,
                              size_t workspace_bytes, void* stream) {
  return wgrad_clip_impl(a, b, B, K, M, N, stride_ab, lda, stride_bb, ldb, layout, dtype, C, clamp,
                         clip_args_dev, out_scale, noise, noise_scale, noise_key, out, ldo,
                         out_dtype, norms, factors, flags, workspace, workspace_bytes, stream,
                         nullptr, 0, nullptr, nullptr, nullptr);
}

namespace {

// Workspace of fdp_wgrad_bias_clip (every part 256-aligned): the weight
// gradient's workspace, the column-sum kernel's (the bias when the generic
// schedule runs), then the bias partials of the grouped and streamed kernels
// (bias_part [B, P, len], bias_sq [B, tiles], sized for both tile grids).
struct BiasLayout {
  size_t wspan, col_off, part_off, sq_off, total;
};
int bias_layout(int64_t B, int64_t K, int64_t M, int64_t N, int dtype, int wflags, int bias_op,
                BiasLayout* l) {
  size_t w = 0, c = 0;
  int st = fdp_wgrad_clip_workspace_size(B, K, M, N, dtype, wflags, &w);
  if (st != FDP_OK) return st;
  st = fdp_colsum_clip_workspace_size(B, K, bias_op == 1 ? M : N, dtype, &c);
  if (st != FDP_OK) return st;
  const int gm = static_cast<int>((M + BM - 1) / BM), gn = static_cast<int>((N + BN - 1) / BN);
  const StreamPlan sp = stream_plan(B, K, M, N, num_cus());
  const int64_t P_group = bias_op == 1 ? gn : gm, P_stream = stream_bias_P(sp, bias_op);
  const int64_t tiles_group = int64_t(gm) * gn, tiles_stream = int64_t(sp.sum_tiles_m) * sp.sum_tiles_n;
  const int64_t P = P_group > P_stream ? P_group : P_stream;
  const int64_t tiles = tiles_group > tiles_stream ? tiles_group : tiles_stream;
  const int64_t len = bias_op == 1 ? M : N;
  l->wspan = align_up(w);
  l->col_off = l->wspan;
  l->part_off = l->col_off + align_up(c);
  l->sq_off = l->part_off + align_up(sizeof(float) * size_t(len) * size_t(B) * size_t(P));
  l->total = l->sq_off + sizeof(float) * size_t(B) * size_t(tiles);
  return FDP_OK;
}

}  // namespace

extern "C" int fdp_wgrad_bias_clip_workspace_size(int64_t B, int64_t K, int64_t M, int64_t N,
                                                  int dtype, int flags, size_t* bytes) {
  if (bytes == nullptr) return FDP_ERR_ARG;
  if (!valid_dtype(dtype)) return FDP_ERR_DTYPE;
  if (B < 1 || M < 1 || N < 1 || K < 0) return FDP_ERR_SHAPE;
  const int bias_op = (flags & FDP_WGRAD_BIAS_OF_B) ? 2 : 1;
  BiasLayout l{};
  const int st = bias_layout(B, K, M, N, dtype, flags & ~FDP_WGRAD_BIAS_OF_B, bias_op, &l);
  if (st != FDP_OK) return st;
  *bytes = l.total;
  return FDP_OK;
}

extern "C" int fdp_wgrad_bias_clip(const void* a, const void* b, int64_t B, int64_t K, int64_t M,
                                   int64_t N, int64_t stride_ab, int64_t lda, int64_t stride_bb,
                                   int64_t ldb, int layout, int dtype, float C, float clamp,
                                   const float* clip_args_dev, float out_scale, const void* noise,
                                   float noise_scale, const fdp_noise_key* noise_key, void* out,
                                   int64_t ldo, int out_dtype, float* norms, float* factors,
                                   int flags, const fdp_bias_out* bias, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  const int bias_op = (flags & FDP_WGRAD_BIAS_OF_B) ? 2 : 1;
  flags &= ~FDP_WGRAD_BIAS_OF_B;
  const int bad = fdp::wgrad_check_args(a, b, B, K, M, N, lda, ldb, layout, dtype, out, ldo,
                                        out_dtype, norms, flags);
  if (bad != FDP_OK) return bad;
  if (bias == nullptr || bias->out == nullptr) return FDP_ERR_ARG;
  if (!valid_dtype(bias->out_dtype)) return FDP_ERR_DTYPE;
  // the bias operand is [B, K, len] over K, contiguous (the column-sum kernel
  // reads it that way when the generic schedule runs); the clip is not
  // optional
  if (layout != FDP_LAYOUT_TN || (flags & FDP_WGRAD_NOCLIP) != 0) return FDP_ERR_ARG;
  if (bias_op == 1 && (lda != M || stride_ab != K * M)) return FDP_ERR_SHAPE;
  if (bias_op == 2 && (ldb != N || stride_bb != K * N)) return FDP_ERR_SHAPE;
  BiasLayout l{};
  int st = bias_layout(B, K, M, N, dtype, flags, bias_op, &l);
  if (st != FDP_OK) return st;
  if (workspace == nullptr || workspace_bytes < l.total) return FDP_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  bool done = false;
  st = wgrad_clip_impl(a, b, B, K, M, N, stride_ab, lda, stride_bb, ldb, layout, dtype, C, clamp,
                       clip_args_dev, out_scale, noise, noise_scale, noise_key, out, ldo,
                       out_dtype, norms, factors, flags, workspace, l.wspan, stream, bias, bias_op,
                       reinterpret_cast<float*>(ws + l.part_off),
                       reinterpret_cast<float*>(ws + l.sq_off), &done);
  if (st != FDP_OK || done) return st;
  return fdp_colsum_clip(bias_op == 1 ? a : b, nullptr, B, K, bias_op == 1 ? M : N, dtype,
                         FDP_NORM_FROB, C, clamp, clip_args_dev, bias->out_scale, bias->noise,
                         bias->noise_scale, bias->noise_key, bias->out, bias->out_dtype,
                         bias->norms, bias->factors, ws + l.col_off, l.part_off - l.col_off,
                         stream);
}
