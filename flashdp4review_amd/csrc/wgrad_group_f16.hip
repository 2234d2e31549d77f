// Grouped single-pass clipped weight-gradient kernel instantiations for f16
// inputs (one translation unit per dtype so that the builds run in parallel).
#include "wgrad_core.hpp"

namespace fdp {
namespace wg {

hipError_t launch_grouped_f16(Args a, int cus, bool plain, bool clean, hipStream_t s) {
  return try_grouped<F16>(a, cus, plain, clean, s);
}

}  // namespace wg
}  // namespace fdp
