// Host side of the input-gradient kernel (dgrad.hpp): plan, argument checks
// and the C entry points fdp_dgrad_workspace_size / fdp_dgrad.
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

constexpr unsigned kSpinLimit = 1u << 24;  // polls of a split's flag (~seconds)
constexpr size_t kAlign = 256;

size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct Plan {
  int bn, tiles_m, tiles_n, splits;
  size_t ticket_off, flag_off, part_off, total;
};

// k-splits (1 or 2) that minimise the estimated time: rounds of workgroups
// over the CUs times the flops of one workgroup's tile; a split adds its
// partial's exchange (x1.06).
Plan make_plan(int64_t M, int64_t N, int64_t K, int cus) {
  Plan pl{};
  pl.bn = kBN;
  pl.tiles_m = static_cast<int>((M + kBM - 1) / kBM);
  pl.tiles_n = static_cast<int>((N + kBN - 1) / kBN);
  const int64_t tiles = int64_t(pl.tiles_m) * pl.tiles_n;
  auto cost = [&](int splits) {
    const int64_t rounds = (tiles * splits + cus - 1) / cus;
    return double(rounds) / splits * (splits > 1 ? 1.06 : 1.0);
  };
  pl.splits = K >= 2 * kBK && cost(2) < cost(1) ? 2 : 1;
  pl.ticket_off = kAlign;  // the status word sits in the first 256 bytes
  pl.flag_off = pl.ticket_off + align_up(sizeof(unsigned) * size_t(tiles));
  pl.part_off = pl.flag_off + align_up(sizeof(unsigned) * size_t(tiles));
  pl.total = pl.part_off +
             (pl.splits > 1 ? sizeof(float) * size_t(tiles) * size_t(kBM) * size_t(kBN) : 0);
  return pl;
}

Plan cached_plan(int64_t M, int64_t N, int64_t K, int cus) {
  static host::ShapeCache<std::tuple<int64_t, int64_t, int64_t, int>, Plan> cache;
  return cache.get(std::make_tuple(M, N, K, cus), [&] { return make_plan(M, N, K, cus); });
}

bool valid16(int dtype) { return dtype == FDP_F16 || dtype == FDP_BF16; }

int check_shape(int64_t M, int64_t N, int64_t K, int layout, int dtype) {
  if (!valid16(dtype)) return FDP_ERR_DTYPE;
  if (layout != FDP_DGRAD_NN && layout != FDP_DGRAD_NT) return FDP_ERR_ARG;
  if (M < 1 || N < 1 || K < kBK || K % kBK != 0) return FDP_ERR_SHAPE;
  if (M > (int64_t(1) << 30) || N > (int64_t(1) << 30)) return FDP_ERR_SHAPE;
  return FDP_OK;
}

}  // namespace
}  // namespace dg
}  // namespace fdp

using fdp::dg::Plan;

extern "C" int fdp_dgrad_workspace_size(int64_t M, int64_t N, int64_t K, int layout, int dtype,
                                        size_t* bytes) {
  if (bytes == nullptr) return FDP_ERR_ARG;
  const int st = fdp::dg::check_shape(M, N, K, layout, dtype);
  if (st != FDP_OK) return st;
  *bytes = fdp::dg::cached_plan(M, N, K, fdp::host::device_cus()).total;
  return FDP_OK;
}

extern "C" int fdp_dgrad(const void* g, const void* w, void* dx, int64_t M, int64_t N, int64_t K,
                         int64_t ldg, int64_t ldw, int64_t ldo, int layout, int dtype,
                         void* workspace, size_t workspace_bytes, void* stream) {
  using namespace fdp::dg;
  int st = check_shape(M, N, K, layout, dtype);
  if (st != FDP_OK) return st;
  if (g == nullptr || w == nullptr || dx == nullptr || workspace == nullptr) return FDP_ERR_ARG;
  const int64_t wrows = layout == FDP_DGRAD_NN ? K : N, wcols = layout == FDP_DGRAD_NN ? N : K;
  if (ldg < K || ldw < wcols || ldo < N) return FDP_ERR_SHAPE;
  // 32-bit buffer records: each operand spans less than 2 GiB
  if (M * ldg * 2 >= (int64_t(1) << 31) || wrows * ldw * 2 >= (int64_t(1) << 31))
    return FDP_ERR_SHAPE;
  if (ldg % 8 != 0 || ldw % 8 != 0 || reinterpret_cast<uintptr_t>(g) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(w) % 16 != 0 || reinterpret_cast<uintptr_t>(dx) % 2 != 0 ||
      reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
    return FDP_ERR_ALIGN;
  const Plan pl = cached_plan(M, N, K, fdp::host::device_cus());
  if (workspace_bytes < pl.total) return FDP_ERR_WORKSPACE;

  char* ws = static_cast<char*>(workspace);
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
  a.splits = pl.splits;
  a.nk = static_cast<int>(K / kBK);
  a.ticket = reinterpret_cast<unsigned*>(ws + pl.ticket_off);
  a.flag = reinterpret_cast<unsigned*>(ws + pl.flag_off);
  a.part = reinterpret_cast<float*>(ws + pl.part_off);
  a.err = reinterpret_cast<int*>(ws);
  a.spin_limit = kSpinLimit;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool wkc = layout == FDP_DGRAD_NT;
  const hipError_t e =
      dtype == FDP_BF16 ? launch_dgrad_bf16(a, wkc, s) : launch_dgrad_f16(a, wkc, s);
  return e == hipSuccess ? FDP_OK : FDP_ERR_HIP;
}
