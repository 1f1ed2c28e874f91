// Instantiations of the dense MaxSim kernel for fp32 tokens (three-term bf16
// split), all features selected at run time.
#include "lik_kernel.h"

namespace lik {
int launch_dense_f32(const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  return launch_dpad<EK_F32, SRC_DENSE, 0, F_ALL>(pl, p, nb, s);
}
}  // namespace lik
