// Instantiations of the dense MaxSim kernel for bf16 tokens at d <= 64 and
// 256 < d <= 512 with the common feature sets compiled to exactly what the
// call uses (the single-query corpus scans of 64- and 512-wide models are
// HBM-bound: the all-features kernel's dead branches cost them a third of
// their bandwidth). Other feature sets go to the generic instantiation.
#include "lik_kernel.h"

namespace lik {
int launch_dense_bf16_generic(const Plan& pl, const Params& p, int64_t nb, hipStream_t s);

int launch_dense_bf16_wide(const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  if (pl.dpad == 64) {
    switch (needed_feat(p)) {
      case 0: return launch_cfg<EK_BF16, 64, SRC_DENSE, 0, 0>(pl, p, nb, s);
      case F_NORMQ: return launch_cfg<EK_BF16, 64, SRC_DENSE, 0, F_NORMQ>(pl, p, nb, s);
      case F_NORM: return launch_cfg<EK_BF16, 64, SRC_DENSE, 0, F_NORM>(pl, p, nb, s);
      default: break;
    }
  } else if (pl.dpad == 512) {
    switch (needed_feat(p)) {
      case 0: return launch_cfg<EK_BF16, 512, SRC_DENSE, 0, 0>(pl, p, nb, s);
      case F_NORMQ: return launch_cfg<EK_BF16, 512, SRC_DENSE, 0, F_NORMQ>(pl, p, nb, s);
      case F_NORM: return launch_cfg<EK_BF16, 512, SRC_DENSE, 0, F_NORM>(pl, p, nb, s);
      default: break;
    }
  }
  return launch_dense_bf16_generic(pl, p, nb, s);
}
}  // namespace lik
