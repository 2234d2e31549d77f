// Grouped single-pass clipped weight-gradient kernel instantiations for bf16
// inputs (one translation unit per dtype so that the builds run in parallel).
#include "wgrad_core.hpp"

namespace fdp {
namespace wg {

hipError_t launch_grouped_bf16(Args a, int cus, bool plain, bool clean, hipStream_t s) {
  return try_grouped<BF16>(a, cus, plain, clean, s);
}

}  // namespace wg
}  // namespace fdp
