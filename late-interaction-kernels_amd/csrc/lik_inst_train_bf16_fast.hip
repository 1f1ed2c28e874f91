// Training-forward (argmax) instantiations of the dense MaxSim kernel for
// bf16 tokens at d = 128 with the common feature sets compiled to exactly
// what the call uses: no doc mask, or prefix / holes masks, with or without
// the query-side normalise (docs arrive normalised by the pre-normalise
// pass), and the in-kernel doc normalise of maxsim_from_hidden. The argmax plans have at least four waves per workgroup, so only
// those column blocks are instantiated. Other calls go to the all-features
// instantiation (lik_inst_train_bf16.hip).
#include "lik_kernel.h"

namespace lik {
int launch_dense_train_bf16_generic(const Plan& pl, const Params& p, int64_t nb, hipStream_t s);

template <int FEAT>
int launch_train_w4(const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  constexpr int F = FEAT | F_ARGMAX;
  if (pl.W == 4 && pl.NSUB == 1) return launch_one<EK_BF16, 128, 4, 1, SRC_DENSE, 0, F>(p, nb, s);
  if (pl.W == 4 && pl.NSUB == 2) return launch_one<EK_BF16, 128, 4, 2, SRC_DENSE, 0, F>(p, nb, s);
  if (pl.W == 8 && pl.NSUB == 1) return launch_one<EK_BF16, 128, 8, 1, SRC_DENSE, 0, F>(p, nb, s);
  if (pl.W == 8 && pl.NSUB == 2) return launch_one<EK_BF16, 128, 8, 2, SRC_DENSE, 0, F>(p, nb, s);
  return launch_dense_train_bf16_generic(pl, p, nb, s);
}

int launch_dense_train_bf16(const Plan& pl, const Params& p, int64_t nb, hipStream_t s) {
  if (pl.dpad == 128) {
    switch (needed_feat(p)) {
      case 0: return launch_train_w4<0>(pl, p, nb, s);
      case F_NORMQ: return launch_train_w4<F_NORMQ>(pl, p, nb, s);
      case F_MASK: return launch_train_w4<F_MASK>(pl, p, nb, s);
      case F_MASK | F_NORMQ: return launch_train_w4<F_MASK | F_NORMQ>(pl, p, nb, s);
      case F_NORM: return launch_train_w4<F_NORM>(pl, p, nb, s);  // docs normalised in the kernel
      default: break;
    }
  }
  return launch_dense_train_bf16_generic(pl, p, nb, s);
}
}  // namespace lik
