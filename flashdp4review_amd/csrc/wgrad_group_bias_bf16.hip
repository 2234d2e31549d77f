// Grouped single-pass kernel instantiations for bf16 inputs that also form the
// bias of operand a or b (Args::bias_op 1 / 2).
#include "wgrad_core.hpp"

namespace fdp {
namespace wg {

hipError_t launch_grouped_bias_bf16(Args a, int cus, bool plain, bool clean, hipStream_t s) {
  return a.bias_op == 1 ? try_grouped<BF16, 1>(a, cus, plain, clean, s)
                        : try_grouped<BF16, 2>(a, cus, plain, clean, s);
}

}  // namespace wg
}  // namespace fdp
