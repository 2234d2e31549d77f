// fdp_noise_advance: the device-side advance of a noise key's counter
// (fdp_noise_key::counter), so that work captured into a HIP graph draws a
// fresh range of the Philox stream on every replay.
#include "fdp_common.hpp"

namespace {

__global__ __launch_bounds__(64) void noise_advance_kernel(uint64_t* counter, uint64_t blocks) {
  if (threadIdx.x == 0 && blockIdx.x == 0) *counter += blocks;
}

}  // namespace

extern "C" int fdp_noise_advance(uint64_t* counter, uint64_t blocks, void* stream) {
  if (counter == nullptr) return FDP_ERR_ARG;
  hipLaunchKernelGGL(noise_advance_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream),
                     counter, blocks);
  return hipGetLastError() == hipSuccess ? FDP_OK : FDP_ERR_HIP;
}
