"""MaxSim (late-interaction) scoring on AMD Instinct MI355X (gfx950).

A drop-in for the ``late_interaction_kernels`` Python API::

    from late_interaction_kernels import maxsim, MaxSimScorer, retrieve

    scores = maxsim(Q, D, q_mask, d_mask, normalize=True)   # [Nq, Nd]
    scores, idx = retrieve(Q, D, top_k=100, chunk=4096)

Every op runs hand-written HIP kernels (bf16/fp16/fp8 MFMA, fused
normalise/mask/PLAID decode, fused top-k merge) from ``_lib/liblik_hip.so``
on the current HIP stream. Inputs must be ROCm GPU tensors. ``maxsim``,
``maxsim_pairs``, the PLAID scorers (in Q) and ``fused_head.maxsim_from_hidden``
are differentiable: an argmax-saving forward plus a deterministic HIP backward.

Submodules mirror the reference: ``forward``, ``score_pairs``, ``padded``,
``plaid``, ``fp8``, ``varlen``, ``topk``, ``retrieve``, ``fused_head``,
``plaid_index``, and ``reference`` (eager PyTorch ground truth for callers'
own comparisons; no op here uses it).
"""

from importlib.metadata import PackageNotFoundError
from importlib.metadata import version as _pkg_version

try:
    __version__ = _pkg_version("late-interaction-kernels-amd")
except PackageNotFoundError:  # running from a source tree
    __version__ = "0.1.0"

from late_interaction_kernels.autograd import maxsim, maxsim_pairs  # noqa: E402
from late_interaction_kernels.padded import maxsim_padded  # noqa: E402
from late_interaction_kernels.retrieve import MaxSimScorer, retrieve  # noqa: E402
from late_interaction_kernels.varlen import maxsim_varlen  # noqa: E402
from late_interaction_kernels import reference  # noqa: E402,F401  (eager PyTorch ground truth)

__all__ = [
    "__version__",
    "MaxSimScorer",
    "retrieve",
    "maxsim_padded",
    "maxsim",
    "maxsim_pairs",
    "maxsim_varlen",
    "reference",
]
