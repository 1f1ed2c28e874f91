"""``maxsim_varlen``: MaxSim on packed (cu_seqlens) inputs (reference varlen.py:452-493)."""

from __future__ import annotations

import torch

from ._core import assert_max_seqlen_covers, packed_maxsim, seqlen_max, unify_dtype
from .autograd import _no_grad_guard


def maxsim_varlen(
    Q_packed: torch.Tensor,
    D_packed: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_d: torch.Tensor,
    max_seqlen_q: int | None = None,
    max_seqlen_d: int | None = None,
) -> torch.Tensor:
    """MaxSim on packed (no-padding) inputs.

    Args:
        Q_packed: ``[sum(Lq_i), d]`` fp16 / bf16 / fp32.
        D_packed: ``[sum(Ld_j), d]``.
        cu_seqlens_q: ``[Nq + 1]`` int32 cumulative offsets.
        cu_seqlens_d: ``[Nd + 1]`` int32 cumulative offsets.
        max_seqlen_q: hard bound on query length (sizes the query block);
            inferred with one device->host sync if omitted, otherwise checked
            by an on-device assert.
        max_seqlen_d: accepted for API compatibility and, when given,
            checked on device; the kernel does not need it (each document's
            tile loop stops at its own length).

    Returns:
        scores ``[Nq, Nd]`` fp32; an empty query or document scores 0.
    """
    if Q_packed.dim() != 2:
        raise ValueError(
            f"Q_packed must be 2-D [sum(Lq_i), d]; got shape {tuple(Q_packed.shape)} "
            f"(ndim={Q_packed.dim()}). For padded inputs use `maxsim(Q, D, ...)` instead."
        )
    if D_packed.dim() != 2:
        raise ValueError(
            f"D_packed must be 2-D [sum(Ld_j), d]; got shape {tuple(D_packed.shape)} "
            f"(ndim={D_packed.dim()}). For padded inputs use `maxsim(Q, D, ...)` instead."
        )
    if D_packed.shape[1] != Q_packed.shape[1]:
        raise ValueError(
            f"Q_packed and D_packed must share the embedding dim; got "
            f"Q_packed.shape[1]={Q_packed.shape[1]} vs D_packed.shape[1]={D_packed.shape[1]}."
        )
    _no_grad_guard(Q_packed, D_packed)
    cu_q = cu_seqlens_q.to(torch.int32).contiguous()
    cu_d = cu_seqlens_d.to(torch.int32).contiguous()
    if max_seqlen_q is None:
        max_seqlen_q = seqlen_max(cu_q)
    else:
        assert_max_seqlen_covers(cu_q, int(max_seqlen_q), "max_seqlen_q")
    if max_seqlen_d is not None:
        assert_max_seqlen_covers(cu_d, int(max_seqlen_d), "max_seqlen_d")
    Qp, Dp = unify_dtype(Q_packed, D_packed)
    return packed_maxsim(Qp, Dp, cu_q, cu_d, int(max_seqlen_q), int(max_seqlen_d or 0))


__all__ = ["maxsim_varlen"]
