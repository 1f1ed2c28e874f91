// Training-forward instantiations of the dense MaxSim kernel for f32 tokens:
// every runtime feature plus the argmax output (F_ARGMAX).
#include "lik_kernel.h"

namespace lik {
int launch_dense_train_f32(const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  return launch_dpad<EK_F32, SRC_DENSE, 0, F_MASK | F_NORM | F_CU | F_ARGMAX>(pl, p, nb, s);
}
}  // namespace lik
