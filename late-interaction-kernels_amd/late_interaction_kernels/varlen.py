"""``maxsim_varlen``: MaxSim on packed (cu_seqlens) inputs (reference varlen.py:452-493),
differentiable in both inputs (reference varlen.py:136-263, 372-449): an
argmax-saving forward and the deterministic HIP backward on packed rows."""

from __future__ import annotations

import torch

from ._core import (assert_max_seqlen_covers, packed_backward, packed_maxsim, packed_maxsim_train, seqlen_max,
                    unify_dtype)
from .autograd import _needs_grad


class _MaxSimVarlenFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, Q, D, cu_q, cu_d, max_q, max_d):
        scores, argmax, Qp, Dp = packed_maxsim_train(Q, D, cu_q, cu_d, max_q, max_d)
        ctx.save_for_backward(Qp, Dp, cu_q, cu_d, argmax)
        ctx.meta = (max_q, max_d, Q.shape[-1], Q.dtype, D.dtype)
        ctx.mark_non_differentiable(argmax)
        return scores

    @staticmethod
    def backward(ctx, grad_scores):
        Qp, Dp, cu_q, cu_d, argmax = ctx.saved_tensors
        max_q, max_d, d, qdt, ddt = ctx.meta
        gq, gd = packed_backward(grad_scores, Qp, Dp, cu_q, cu_d, argmax, max_q, max_d,
                                 need_d=ctx.needs_input_grad[1])
        gq = gq[:, :d].to(qdt) if ctx.needs_input_grad[0] else None
        gd = gd[:, :d].to(ddt) if gd is not None else None
        return gq, gd, None, None, None, None


def maxsim_varlen(
    Q_packed: torch.Tensor,
    D_packed: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_d: torch.Tensor,
    max_seqlen_q: int | None = None,
    max_seqlen_d: int | None = None,
) -> torch.Tensor:
    """MaxSim on packed (no-padding) inputs. Autograd-aware.

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
    cu_q = cu_seqlens_q.to(torch.int32).contiguous()
    cu_d = cu_seqlens_d.to(torch.int32).contiguous()
    if max_seqlen_q is None:
        max_seqlen_q = seqlen_max(cu_q)
    else:
        assert_max_seqlen_covers(cu_q, int(max_seqlen_q), "max_seqlen_q")
    if max_seqlen_d is not None:
        assert_max_seqlen_covers(cu_d, int(max_seqlen_d), "max_seqlen_d")
    Qp, Dp = unify_dtype(Q_packed, D_packed)
    if _needs_grad(Q_packed, D_packed):
        if Qp.dtype == torch.float64:
            raise TypeError("maxsim_varlen gradients support fp16 / bf16 / fp32 inputs")
        # the backward's grid over packed doc rows is sized by the longest doc
        max_d = seqlen_max(cu_d) if max_seqlen_d is None else int(max_seqlen_d)
        return _MaxSimVarlenFn.apply(Qp, Dp, cu_q, cu_d, int(max_seqlen_q), max_d)
    return packed_maxsim(Qp, Dp, cu_q, cu_d, int(max_seqlen_q), int(max_seqlen_d or 0))


__all__ = ["maxsim_varlen"]
