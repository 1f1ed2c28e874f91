"""Chunked top-k MaxSim (reference topk.py:12-91), with a fused HIP merge.

Each document chunk is scored by the MaxSim kernel into a ``[Nq, chunk]``
buffer, then ``lik_topk_select`` folds it into the running ``[Nq, k]`` list
in one call, however wide the chunk (a tree of workgroups for wide rows).
Ties are broken by the lower document index, so chunked and unchunked calls
return identical results (torch.topk leaves tie order unspecified).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._core import dense_maxsim, unify_dtype

TOPK_MAX_K = 8192  # largest k the fused select handles


def _merge_sorted_fallback(s, i, k, largest):
    # k > TOPK_MAX_K: stable sort keeps (prev, then chunk) order among equal
    # scores, which is ascending index order -> same tie rule as the kernel.
    order = torch.sort(s, dim=-1, descending=largest, stable=True).indices[:, :k]
    return torch.gather(s, -1, order), torch.gather(i, -1, order)


def topk_update(
    chunk_scores: torch.Tensor,
    idx_base: int,
    run_s: torch.Tensor | None,
    run_i: torch.Tensor | None,
    k: int,
    largest: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Merge ``chunk_scores [R, n]`` (doc indices ``idx_base + c``) into the
    running top-k ``(run_s, run_i)``; returns the new running list of width
    ``min(k, prev_width + n)``, best first."""
    _lib.require_gpu(chunk_scores)
    R, n = chunk_scores.shape
    dev = chunk_scores.device
    if k > TOPK_MAX_K:
        idx = torch.arange(idx_base, idx_base + n, device=dev, dtype=torch.int64).expand(R, n)
        if run_s is None:
            s_all, i_all = chunk_scores, idx
        else:
            s_all, i_all = torch.cat([run_s, chunk_scores], -1), torch.cat([run_i, idx], -1)
        return _merge_sorted_fallback(s_all, i_all, min(k, s_all.shape[-1]), largest)
    lib = _lib.load()
    cs = chunk_scores.contiguous() if chunk_scores.stride(-1) != 1 else chunk_scores
    pk = 0 if run_s is None else run_s.shape[-1]
    kk = min(k, pk + n)
    out_s = torch.empty(R, kk, device=dev, dtype=torch.float32)
    out_i = torch.empty(R, kk, device=dev, dtype=torch.int64)
    if R == 0 or kk == 0:
        return out_s, out_i
    nws = lib.lik_topk_select_workspace_size(R, n, kk)
    ws = torch.empty(nws, device=dev, dtype=torch.uint8) if nws else None
    with torch.cuda.device(dev):
        rc = lib.lik_topk_select(
            cs.data_ptr(), R, n, cs.stride(0), idx_base,
            _lib.ptr(run_s), _lib.ptr(run_i), pk, run_s.stride(0) if run_s is not None else 0,
            kk, 1 if largest else 0, out_s.data_ptr(), out_i.data_ptr(), kk, _lib.ptr(ws), nws,
            _lib.stream_of(out_s),
        )
    _lib.check(rc, "lik_topk_select")
    return out_s, out_i


def maxsim_topk(
    Q: torch.Tensor,
    D: torch.Tensor,
    k: int,
    q_mask: torch.Tensor | None = None,
    d_mask: torch.Tensor | None = None,
    *,
    normalize: bool = False,
    chunk_size: int | None = None,
    largest: bool = True,
    sorted: bool = True,  # noqa: A002 - reference kwarg name
) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-``k`` documents per query: ``(scores [Nq, k], indices [Nq, k])``.

    ``k`` is clamped to ``Nd``. Results are always sorted best-first (valid
    for ``sorted=False`` too) with ties broken by the lower index.
    """
    if k <= 0:
        raise ValueError(f"k must be positive, got {k}")
    q_was_2d = Q.dim() == 2
    if q_was_2d:
        Q = Q.unsqueeze(0)
    if D.dim() == 2:
        D = D.unsqueeze(0)
    if q_mask is not None and q_mask.dim() == 1:
        q_mask = q_mask.unsqueeze(0)
    if d_mask is not None and d_mask.dim() == 1:
        d_mask = d_mask.unsqueeze(0)
    if Q.shape[-1] != D.shape[-1]:
        raise ValueError(f"Q and D must share the embedding dim; got {Q.shape[-1]} vs {D.shape[-1]}.")
    Q, D = unify_dtype(Q, D)
    Nq = Q.shape[0]
    Nd = D.shape[0]
    k = min(k, Nd)
    if Nd == 0:
        e = torch.empty(Nq, 0, device=Q.device)
        return (e.squeeze(0), e.long().squeeze(0)) if q_was_2d else (e, e.long())
    cs = Nd if chunk_size is None or chunk_size >= Nd else int(chunk_size)
    if cs <= 0:
        raise ValueError(f"chunk must be positive, got {chunk_size}")
    run_s = run_i = None
    with torch.no_grad():
        for start in range(0, Nd, cs):
            end = min(start + cs, Nd)
            dm = d_mask[start:end] if d_mask is not None else None
            s = dense_maxsim(Q, D[start:end], q_mask, dm, normalize=normalize)
            run_s, run_i = topk_update(s, start, run_s, run_i, k, largest)
    if q_was_2d:
        return run_s.squeeze(0), run_i.squeeze(0)
    return run_s, run_i


__all__ = ["maxsim_topk", "topk_update"]
