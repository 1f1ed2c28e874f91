// Instantiations of the PLAID decode+MaxSim kernel computing in f16, for
// bf16 / fp16 / fp32 centroid tables.
#include "lik_kernel.h"

namespace lik {
int launch_plaid_f16(int cd, const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  if (pl.dpad > 256) return LIK_ERR_UNSUPPORTED;
  if (cd == LIK_BF16) return launch_dpad<EK_F16, SRC_PLAID, EK_BF16, 0>(pl, p, nb, s);
  if (cd == LIK_F16) return launch_dpad<EK_F16, SRC_PLAID, EK_F16, 0>(pl, p, nb, s);
  if (cd == LIK_F32) return launch_dpad<EK_F16, SRC_PLAID, EK_F32, 0>(pl, p, nb, s);
  return LIK_ERR_UNSUPPORTED;
}
}  // namespace lik
