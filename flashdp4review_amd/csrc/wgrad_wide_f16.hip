// Wide single-pass kernel instantiations for f16 inputs (one translation unit
// per dtype so that the builds run in parallel).
#include "wgrad_wide.hpp"

namespace fdp {
namespace wg {

hipError_t launch_wide_f16(const WideArgs& a, int wgm, bool plain, hipStream_t s) {
  return launch_wide_t<F16>(a, wgm, plain, s);
}

}  // namespace wg
}  // namespace fdp
