// Two-pass (Gram norm + streamed clipped sum) kernel instantiations for bf16
// inputs.
#include "wgrad_stream.hpp"

namespace fdp {
namespace wg {

hipError_t launch_gram_norm_bf16(const GramArgs& g, hipStream_t s) {
  return launch_gram_norm<BF16>(g, s);
}
hipError_t launch_clipsum_bf16(const Args& a, const StreamPlan& sp, hipStream_t s) {
  return launch_clipsum<BF16>(a, sp, s);
}

}  // namespace wg
}  // namespace fdp
