// Instantiations of the dense MaxSim kernel for bf16 tokens at d <= 128 with
// the feature set compiled to exactly what the call uses (fewer live scalars,
// no dead branches in the tile loop). Anything else goes to the generic
// instantiation.
#include "lik_kernel.h"

namespace lik {
int launch_dense_bf16_generic(const Plan& pl, const Params& p, int64_t nb, hipStream_t s);
int launch_dense_bf16_wide(const Plan& pl, const Params& p, int64_t nb, hipStream_t s);

int launch_dense_bf16(const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  if (pl.dpad == 128) {
    switch (needed_feat(p)) {
    case 0: return launch_cfg<EK_BF16, 128, SRC_DENSE, 0, 0>(pl, p, nb, s);
    case F_MASK: return launch_cfg<EK_BF16, 128, SRC_DENSE, 0, F_MASK>(pl, p, nb, s);
    case F_NORM: return launch_cfg<EK_BF16, 128, SRC_DENSE, 0, F_NORM>(pl, p, nb, s);
    case F_MASK | F_NORM: return launch_cfg<EK_BF16, 128, SRC_DENSE, 0, F_MASK | F_NORM>(pl, p, nb, s);
    case F_CU: return launch_cfg<EK_BF16, 128, SRC_DENSE, 0, F_CU>(pl, p, nb, s);
    case F_CU | F_NORM: return launch_cfg<EK_BF16, 128, SRC_DENSE, 0, F_CU | F_NORM>(pl, p, nb, s);
    case F_NORMQ: return launch_cfg<EK_BF16, 128, SRC_DENSE, 0, F_NORMQ>(pl, p, nb, s);
    case F_MASK | F_NORMQ: return launch_cfg<EK_BF16, 128, SRC_DENSE, 0, F_MASK | F_NORMQ>(pl, p, nb, s);
    case F_CU | F_NORMQ: return launch_cfg<EK_BF16, 128, SRC_DENSE, 0, F_CU | F_NORMQ>(pl, p, nb, s);
      default: break;
    }
  }
  if (pl.dpad == 64 || pl.dpad == 512) return launch_dense_bf16_wide(pl, p, nb, s);
  return launch_dense_bf16_generic(pl, p, nb, s);
}
}  // namespace lik
