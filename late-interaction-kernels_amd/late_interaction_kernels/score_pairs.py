"""``score_pairs_packed``: MaxSim over an explicit (query, doc) pair list
(reference score_pairs.py:423-511), on packed inputs."""

from __future__ import annotations

import torch

from ._core import assert_max_seqlen_covers, pairs_maxsim, seqlen_max, unify_dtype
from .autograd import _no_grad_guard


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

    Returns ``[num_pairs]`` fp32. Pairs whose query or document is empty
    (or whose index is out of range) score 0. Query length is bounded by
    the kernel's query block (512 tokens for d <= 128).
    """
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
    return pairs_maxsim(Qp, Dp, cu_q, cu_d, pair_q_idx, pair_d_idx, int(max_seqlen_q), int(max_seqlen_d or 0))


__all__ = ["score_pairs_packed"]
