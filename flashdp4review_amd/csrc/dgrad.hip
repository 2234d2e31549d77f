// Host side of the input-gradient kernel (dgrad.hpp): plan, argument checks
// and the C entry point fdp_dgrad.
//
// Reference: the grad_input products of the DP layers' backward,
// flashdp/layers/linear.py:62-67 (grad_output @ weight) and
// flashdp/layers/transformers_conv1d.py:70-77 (grad_output @ weight.t()),
// which the reference leaves to torch's matmul.
#include "dgrad.hpp"
#include "host_cache.hpp"

namespace fdp {
namespace dg {
namespace {

struct Plan {
  int bm, tiles_m, tiles_n;
};

// Tile height (256 or 128 rows of g) that needs the fewer rounds of
// workgroups over the CUs, each round weighted by its tile's rows and the
// 128-row tile by x1.15 (its waves hold 32 rows: fewer MFMAs per fragment
// read; measured at cfg3's shape, where 256 rows fill the CUs in one round).
Plan make_plan(int64_t M, int64_t N, int cus) {
  Plan pl{};
  const int64_t tn = (N + kBN - 1) / kBN;
  double best = 0.0;
  for (int bm : {kBM, kBMHalf}) {
    const int64_t tm = (M + bm - 1) / bm;
    const int64_t rounds = (tm * tn + cus - 1) / cus;
    const double cost = double(rounds) * bm * (bm == kBMHalf ? 1.15 : 1.0);
    if (best == 0.0 || cost < best) {
      best = cost;
      pl.bm = bm;
      pl.tiles_m = static_cast<int>(tm);
      pl.tiles_n = static_cast<int>(tn);
    }
  }
  return pl;
}

Plan cached_plan(int64_t M, int64_t N, int cus) {
  static host::ShapeCache<std::tuple<int64_t, int64_t, int>, Plan> cache;
  return cache.get(std::make_tuple(M, N, cus), [&] { return make_plan(M, N, cus); });
}

}  // namespace
}  // namespace dg
}  // namespace fdp

extern "C" int fdp_dgrad(const void* g, const void* w, void* dx, int64_t M, int64_t N, int64_t K,
                         int64_t ldg, int64_t ldw, int64_t ldo, int layout, int dtype,
                         void* stream) {
  using namespace fdp::dg;
  if (dtype != FDP_F16 && dtype != FDP_BF16) return FDP_ERR_DTYPE;
  if (layout != FDP_DGRAD_NN && layout != FDP_DGRAD_NT) return FDP_ERR_ARG;
  if (M < 1 || N < 1 || K < kBK || K % kBK != 0) return FDP_ERR_SHAPE;
  if (M > (int64_t(1) << 30) || N > (int64_t(1) << 30)) return FDP_ERR_SHAPE;
  if (g == nullptr || w == nullptr || dx == nullptr) return FDP_ERR_ARG;
  const int64_t wrows = layout == FDP_DGRAD_NN ? K : N, wcols = layout == FDP_DGRAD_NN ? N : K;
  if (ldg < K || ldw < wcols || ldo < N) return FDP_ERR_SHAPE;
  // 32-bit buffer records: each operand spans less than 2 GiB
  if (!fdp::fits_record(M, ldg) || !fdp::fits_record(wrows, ldw)) return FDP_ERR_SHAPE;
  if (ldg % 8 != 0 || ldw % 8 != 0 || reinterpret_cast<uintptr_t>(g) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(w) % 16 != 0 || reinterpret_cast<uintptr_t>(dx) % 2 != 0)
    return FDP_ERR_ALIGN;
  const Plan pl = cached_plan(M, N, fdp::host::device_cus());
  if (int64_t(pl.tiles_m) * pl.tiles_n >= (int64_t(1) << 30)) return FDP_ERR_SHAPE;  // grid size

  DgradArgs a{};
  a.g = static_cast<const uint16_t*>(g);
  a.w = static_cast<const uint16_t*>(w);
  a.out = static_cast<uint16_t*>(dx);
  a.vec_out = ldo % 8 == 0 && reinterpret_cast<uintptr_t>(dx) % 16 == 0;
  a.M = M;
  a.N = N;
  a.K = K;
  a.ldg = ldg;
  a.ldw = ldw;
  a.ldo = ldo;
  a.tiles_m = pl.tiles_m;
  a.tiles_n = pl.tiles_n;
  a.nk = static_cast<int>(K / kBK);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool wkc = layout == FDP_DGRAD_NT;
  const hipError_t e = dtype == FDP_BF16 ? launch_dgrad_bf16(a, pl.bm, wkc, s)
                                         : launch_dgrad_f16(a, pl.bm, wkc, s);
  return e == hipSuccess ? FDP_OK : FDP_ERR_HIP;
}
