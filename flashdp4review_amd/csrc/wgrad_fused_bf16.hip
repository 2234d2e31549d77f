// Single-pass clipped weight-gradient kernel instantiations for bf16 inputs
// (one translation unit per dtype so that the builds run in parallel).
#include "wgrad_core.hpp"

namespace fdp {
namespace wg {

hipError_t launch_fused_bf16(Args a, int cus, hipStream_t s) {
  return try_fused<Core16<BF16>>(a, cus, kMaxUnits16, s);
}

}  // namespace wg
}  // namespace fdp
