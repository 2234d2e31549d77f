// Single-pass clipped weight-gradient kernel instantiations for f32 inputs
// (one translation unit per dtype so that the builds run in parallel).
#include "wgrad_core.hpp"

namespace fdp {
namespace wg {

hipError_t launch_fused_f32(Args a, int cus, hipStream_t s) {
  return try_fused<Core32>(a, cus, kMaxUnits32, s);
}

}  // namespace wg
}  // namespace fdp
