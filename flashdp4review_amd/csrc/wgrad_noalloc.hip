// fdp_wgrad_clip_noalloc: the clipped per-sample product sum for callers that
// cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc).  It is fdp_wgrad_clip with its
// workspace taken from `scratch`, a file-scope device array of
// FDP_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds until the
// process ends, instead of a caller-provided buffer.
//
//  * Set-up: on the first call on a device (with that device current) the
//    array's device address is taken with hipGetSymbolAddress and kept per
//    device; each GPU holds its own copy at its own address.  Host code uses
//    only that address (the array's name is a host-side stand-in).
//  * The call allocates nothing (no hipMalloc / hipFree, no allocating
//    library routine) and always uses the ordinary (non-cooperative) launch.
//  * State: every call clears the control words at the array's head with a
//    fill kernel (no hipMemsetAsync), and the kernels rewrite or clear
//    everything else they read, so leftovers of the previous call do not
//    matter.  All calls on one GPU share the array: calls that overlap on one
//    GPU (other streams, other threads) race and must be serialised by the
//    caller.
//  * Problems whose workspace exceeds the array are rejected with
//    FDP_ERR_TOO_LARGE before anything is launched; a stream of another
//    device than the current one with FDP_ERR_ARG.
#include <mutex>

#include "fdp_common.hpp"

namespace {

static __device__ __align__(256) unsigned char scratch[FDP_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};

// This device's copy of `scratch` (nullptr if it cannot be resolved).
void* device_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> g(g_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      return nullptr;
    }
    g_scratch[dev] = p;
  }
  return g_scratch[dev];
}

}  // namespace

extern "C" int fdp_wgrad_clip_noalloc(const void* a, const void* b, int64_t B, int64_t K,
                                      int64_t M, int64_t N, int64_t stride_ab, int64_t lda,
                                      int64_t stride_bb, int64_t ldb, int layout, int dtype,
                                      float C, float clamp, const float* clip_args_dev,
                                      float out_scale, const void* noise, float noise_scale,
                                      const fdp_noise_key* noise_key, void* out, int64_t ldo,
                                      int out_dtype, float* norms, float* factors, int flags,
                                      void* stream) {
  const int bad = fdp::wgrad_check_args(a, b, B, K, M, N, lda, ldb, layout, dtype, out, ldo,
                                        out_dtype, norms, flags);
  if (bad != FDP_OK) return bad;
  // The scratch copy, the plan (CU count) and the launch are those of the
  // current device: the stream must belong to it.
  if (stream != nullptr) {
    int cur = 0;
    hipDevice_t sd = 0;
    if (hipGetDevice(&cur) != hipSuccess ||
        hipStreamGetDevice(static_cast<hipStream_t>(stream), &sd) != hipSuccess) {
      (void)hipGetLastError();
      return FDP_ERR_ARG;
    }
    if (static_cast<int>(sd) != cur) return FDP_ERR_ARG;
  }
  // The control words are cleared by the call itself (a small fill kernel):
  // an expired wait of an earlier call may have left its status word set.
  flags = (flags | FDP_WGRAD_PLAIN_LAUNCH) & ~FDP_WGRAD_CLEAN_WORKSPACE;
  size_t need = 0;
  const int st = fdp_wgrad_clip_workspace_size(B, K, M, N, dtype, flags, &need);
  if (st != FDP_OK) return st;
  if (need > size_t(FDP_NOALLOC_SCRATCH_BYTES)) return FDP_ERR_TOO_LARGE;
  void* ws = device_scratch();
  if (ws == nullptr) return FDP_ERR_HIP;
  return fdp_wgrad_clip(a, b, B, K, M, N, stride_ab, lda, stride_bb, ldb, layout, dtype, C, clamp,
                        clip_args_dev, out_scale, noise, noise_scale, noise_key, out, ldo,
                        out_dtype, norms, factors, flags, ws, size_t(FDP_NOALLOC_SCRATCH_BYTES),
                        stream);
}
