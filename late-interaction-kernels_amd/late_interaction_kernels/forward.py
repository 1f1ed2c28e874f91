"""``maxsim_forward``: the low-level forward entry point.

Same signature and return convention as the reference's
``forward.maxsim_forward`` (``forward.py:349-398``): ``(scores, argmax)``
with ``scores`` ``[Nq, Nd]`` fp32 (squeezed like ``maxsim`` for 2-D
inputs) and ``argmax`` the ``[Nq * Nd, Lq]`` int32 winning doc-token index
per (query, doc, query token) when ``save_argmax`` is set, else ``None``.
Ties go to the lowest doc-token index and ``-1`` marks a query token whose
max ranges over no valid doc token. No autograd: it is the raw kernel call
that ``maxsim`` wraps (``lik_maxsim`` / ``lik_maxsim_argmax``).
"""

from __future__ import annotations

import torch

from ._core import dense_maxsim, dense_maxsim_train, unify_dtype


def maxsim_forward(
    Q: torch.Tensor,
    D: torch.Tensor,
    q_mask: torch.Tensor | None = None,
    d_mask: torch.Tensor | None = None,
    *,
    save_argmax: bool = False,
    normalize: bool = False,
):
    """Fused MaxSim forward over ``Q [Nq, Lq, d]`` (or ``[Lq, d]``) and
    ``D [Nd, Ld, d]`` (or ``[Ld, d]``); masks are ``True`` = keep."""
    q2, d2 = Q.dim() == 2, D.dim() == 2
    if q2:
        Q = Q.unsqueeze(0)
    if d2:
        D = D.unsqueeze(0)
    if q_mask is not None and q_mask.dim() == 1:
        q_mask = q_mask.unsqueeze(0)
    if d_mask is not None and d_mask.dim() == 1:
        d_mask = d_mask.unsqueeze(0)
    if Q.dim() != 3 or D.dim() != 3:
        raise ValueError(f"maxsim_forward expects Q [Nq, Lq, d] and D [Nd, Ld, d]; got {tuple(Q.shape)}, "
                         f"{tuple(D.shape)}")
    if Q.shape[-1] != D.shape[-1]:
        raise ValueError(f"embedding dims don't match: Q has d={Q.shape[-1]}, D has d={D.shape[-1]}")
    Qc, Dc = unify_dtype(Q, D)
    norm = 3 if normalize else 0
    if save_argmax:
        scores, argmax, *_ = dense_maxsim_train(Qc.detach(), Dc.detach(), q_mask, d_mask, norm=norm, kd=False)
    else:
        scores, argmax = dense_maxsim(Qc, Dc, q_mask, d_mask, norm=norm), None
    if q2 and d2:
        return scores.reshape(()), argmax
    if q2:
        return scores.squeeze(0), argmax
    if d2:
        return scores.squeeze(-1), argmax
    return scores, argmax


__all__ = ["maxsim_forward"]
