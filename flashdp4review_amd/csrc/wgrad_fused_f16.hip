// Single-pass clipped weight-gradient kernel instantiations for f16 inputs
// (one translation unit per dtype so that the builds run in parallel).
#include "wgrad_core.hpp"

namespace fdp {
namespace wg {

hipError_t launch_fused_f16(Args a, int cus, hipStream_t s) {
  return try_fused<Core16<F16>>(a, cus, kMaxUnits16, s);
}

}  // namespace wg
}  // namespace fdp
