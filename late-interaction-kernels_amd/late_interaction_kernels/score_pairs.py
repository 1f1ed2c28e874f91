"""``score_pairs_packed``: MaxSim over an explicit (query, doc) pair list
(reference score_pairs.py:423-511), on packed inputs. Differentiable in both
inputs (reference score_pairs.py:344-420): argmax-saving forward and the
deterministic pair-list backward."""

from __future__ import annotations

import torch

from ._core import (assert_max_seqlen_covers, pairs_backward, pairs_maxsim, pairs_maxsim_train, seqlen_max,
                    unify_dtype)
from .autograd import _needs_grad


class _ScorePairsFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, Q, D, cu_q, cu_d, pair_q, pair_d, max_q, max_d):
        scores, argmax, Qp, Dp = pairs_maxsim_train(Q, D, cu_q, cu_d, pair_q, pair_d, max_q, max_d)
        ctx.save_for_backward(Qp, Dp, cu_q, cu_d, pair_q, pair_d, argmax)
        ctx.meta = (max_q, max_d, Q.shape[-1], Q.dtype, D.dtype)
        ctx.mark_non_differentiable(argmax)
        return scores

    @staticmethod
    def backward(ctx, grad_scores):
        Qp, Dp, cu_q, cu_d, pair_q, pair_d, argmax = ctx.saved_tensors
        max_q, max_d, d, qdt, ddt = ctx.meta
        gq, gd = pairs_backward(grad_scores, Qp, Dp, cu_q, cu_d, pair_q, pair_d, argmax, max_q, max_d,
                                need_d=ctx.needs_input_grad[1])
        gq = gq[:, :d].to(qdt) if ctx.needs_input_grad[0] else None
        gd = gd[:, :d].to(ddt) if gd is not None else None
        return gq, gd, None, None, None, None, None, None


def score_pairs_packed(
    Q_packed: torch.Tensor,
    D_packed: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_d: torch.Tensor,
    pair_q_idx: torch.Tensor,
    pair_d_idx: torch.Tensor,
    *,
    max_seqlen_q: int | None = None,
    max_seqlen_d: int | None = None,
) -> torch.Tensor:
    """``scores[k] = MaxSim(Q_packed[cu_q[pq[k]]:cu_q[pq[k]+1]], D_packed[cu_d[pd[k]]:...])``.

    Autograd-aware. Returns ``[num_pairs]`` fp32. Pairs whose query or document is empty
    (or whose index is out of range) score 0. Any query length (queries longer
    than the kernel's 512-token query block are scored in token chunks whose
    partial sums are added in order) and any embedding dim (rows wider than
    512 take the one-wave-per-pair kernel)."""
    if Q_packed.dim() != 2 or D_packed.dim() != 2:
        raise ValueError(
            "Q_packed / D_packed must be 2-D [sum(L), d]; "
            f"got Q={tuple(Q_packed.shape)}, D={tuple(D_packed.shape)}."
        )
    if D_packed.shape[1] != Q_packed.shape[1]:
        raise ValueError(f"Q / D embedding dims mismatch: {Q_packed.shape[1]} vs {D_packed.shape[1]}.")
    if pair_q_idx.shape != pair_d_idx.shape or pair_q_idx.dim() != 1:
        raise ValueError(
            f"pair_q_idx / pair_d_idx must be matching 1-D tensors; "
            f"got {tuple(pair_q_idx.shape)} vs {tuple(pair_d_idx.shape)}."
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
            raise TypeError("score_pairs_packed gradients support fp16 / bf16 / fp32 inputs")
        max_d = seqlen_max(cu_d) if max_seqlen_d is None else int(max_seqlen_d)  # sizes the grad_D grid
        pq = pair_q_idx.to(device=Qp.device, dtype=torch.int32).contiguous()
        pd = pair_d_idx.to(device=Qp.device, dtype=torch.int32).contiguous()
        return _ScorePairsFn.apply(Qp, Dp, cu_q, cu_d, pq, pd, int(max_seqlen_q), max_d)
    return pairs_maxsim(Qp, Dp, cu_q, cu_d, pair_q_idx, pair_d_idx, int(max_seqlen_q), int(max_seqlen_d or 0))


__all__ = ["score_pairs_packed"]
