// Input-gradient (dX) kernel instantiations for f16 operands (one translation
// unit per dtype so that the builds run in parallel).
#include "dgrad.hpp"

namespace fdp {
namespace dg {

hipError_t launch_dgrad_f16(const DgradArgs& a, int bm, bool wkc, hipStream_t s) {
  return launch_dgrad_t<F16>(a, bm, wkc, s);
}

}  // namespace dg
}  // namespace fdp
