// Instantiations of the dense MaxSim kernel for fp8 tokens, all features
// selected at run time (FEAT = F_ALL).
#include "lik_kernel.h"

namespace lik {
int launch_dense_fp8_generic(const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  return launch_dpad<EK_FP8, SRC_DENSE, 0, F_ALL>(pl, p, nb, s);
}
}  // namespace lik
