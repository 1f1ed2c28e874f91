// Training-forward instantiations of the dense MaxSim kernel for bf16 tokens:
// every runtime feature plus the argmax output (F_ARGMAX); the common d = 128
// feature sets have their own (lik_inst_train_bf16_fast.hip).
#include "lik_kernel.h"

namespace lik {
int launch_dense_train_bf16_generic(const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  return launch_dpad<EK_BF16, SRC_DENSE, 0, F_MASK | F_NORM | F_CU | F_ARGMAX>(pl, p, nb, s);
}
}  // namespace lik
