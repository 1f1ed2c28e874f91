"""``maxsim_from_hidden``: MaxSim with the doc-side projection head in front
(reference fused_head.py:262-332).

Computes ``maxsim(Q, normalize(F.linear(H_d, W, b)))`` with the doc-token
normalisation done inside the MaxSim kernel (``LIK_NORMALIZE_D``; Q is taken
as already projected and normalised, as in the reference). The projection is a
plain GEMM, left to hipBLASLt through ``F.linear``; the reference fuses it into
its Triton kernel to avoid materialising ``D``, which at MI355X's 288 GB costs
``Nd * Ld * d_out`` elements of scratch. Gradients flow into ``Q``, ``H_d``,
``W`` and ``b`` (MaxSim backward in HIP, the projection's in hipBLASLt).
"""

from __future__ import annotations

import torch

from .autograd import _score, _validate_devices
from ._core import unify_dtype


def maxsim_from_hidden(
    Q: torch.Tensor,
    H_d: torch.Tensor,
    W: torch.Tensor,
    b: torch.Tensor | None = None,
    d_mask: torch.Tensor | None = None,
    normalize: bool = True,
) -> torch.Tensor:
    """``Q [Lq, d_out] | [Nq, Lq, d_out]``, ``H_d [Nd, Ld, d_model]``, ``W [d_out, d_model]``,
    ``b [d_out]`` -> fp32 scores ``[Nq, Nd]`` (``[Nd]`` for 2-D Q)."""
    q_was_2d = Q.dim() == 2
    if q_was_2d:
        Q = Q.unsqueeze(0)
    if d_mask is not None and d_mask.dim() == 1:
        d_mask = d_mask.unsqueeze(0)
    if Q.dim() != 3:
        raise ValueError(f"Q must be [Lq, d_out] or [Nq, Lq, d_out]; got {Q.shape}")
    if H_d.dim() != 3:
        raise ValueError(f"H_d must be [Nd, Ld, d_model]; got {H_d.shape}")
    if W.dim() != 2 or W.shape != (Q.shape[-1], H_d.shape[-1]):
        raise ValueError(f"W must be [d_out={Q.shape[-1]}, d_model={H_d.shape[-1]}]; got {W.shape}")
    if Q.device != H_d.device or W.device != Q.device:
        raise ValueError("Q, H_d, W must be on the same device.")
    if b is not None and (b.dim() != 1 or b.shape[0] != Q.shape[-1]):
        raise ValueError(f"b must be [d_out={Q.shape[-1]}]; got {tuple(b.shape) if b is not None else None}")
    _validate_devices(Q, H_d, None, d_mask)
    D = torch.nn.functional.linear(H_d, W, b)
    Q, D = unify_dtype(Q, D)
    scores = _score(Q, D, None, d_mask, normalize=2 if normalize else 0)
    return scores.squeeze(0) if q_was_2d else scores


__all__ = ["maxsim_from_hidden"]
