"""Eager PyTorch ground truth for MaxSim: the public ``reference`` submodule.

The reference package exports this module by name (``__init__.py:65``) so
that downstream tests can compare its kernels against plain PyTorch. The same
functions, signatures and results are provided here; they run wherever
PyTorch runs (CPU or GPU tensors) and compute in fp32 (fp64 inputs stay
fp64). They are slow by design.

No op of this package calls these functions: every scoring entry point runs
the HIP kernels and raises when they are unavailable. This module is only for
callers who want an independent eager result to compare with.

Score: ``score[i, j] = sum_{s kept in q_mask} max_{t kept in d_mask} <Q[i, s], D[j, t]>``;
a max over no kept doc token (or a non-finite max) contributes 0, and
``normalize`` divides each token by ``max(||x||, 1e-12)``
(reference ``reference.py:26-98``). Instead of materialising the full
``[Nq, Nd, Lq, Ld]`` similarity tensor, the dense functions walk query
blocks so the temporary stays below about 256 MB.
"""

from __future__ import annotations

import torch

NEG_INF = float("-inf")
_BLOCK_ELEMS = 1 << 26  # similarity elements per query block


def _widen(x: torch.Tensor) -> torch.Tensor:
    """fp16 / bf16 / fp8 -> fp32; fp32 and fp64 unchanged."""
    return x if x.dtype in (torch.float32, torch.float64) else x.float()


def _unit(x: torch.Tensor) -> torch.Tensor:
    return torch.nn.functional.normalize(x, p=2, dim=-1, eps=1e-12)


def _row_max_sum(Q: torch.Tensor, D: torch.Tensor, q_keep, d_keep, *, finite_only: bool = True) -> torch.Tensor:
    """Masked MaxSim of Q [Nq, Lq, d] against D [Nd, Ld, d] -> [Nq, Nd].
    ``finite_only``: a non-finite row max counts 0 (else only a max over no
    kept doc token does)."""
    Nq, Lq, d = Q.shape
    Nd, Ld, _ = D.shape
    dtype = torch.promote_types(Q.dtype, D.dtype)
    out = torch.zeros(Nq, Nd, dtype=dtype, device=Q.device)
    if Nq == 0 or Nd == 0 or Lq == 0 or Ld == 0:
        return out
    Dflat = D.reshape(Nd * Ld, d).to(dtype)
    step = max(1, _BLOCK_ELEMS // max(1, Lq * Nd * Ld))
    for i0 in range(0, Nq, step):
        i1 = min(Nq, i0 + step)
        sim = (Q[i0:i1].reshape(-1, d).to(dtype) @ Dflat.T).view(i1 - i0, Lq, Nd, Ld)
        if d_keep is not None:
            sim = sim.masked_fill(~d_keep[None, None], NEG_INF)
        best = sim.amax(dim=-1)  # [b, Lq, Nd]
        if finite_only:
            best = torch.where(torch.isfinite(best), best, torch.zeros_like(best))
        elif d_keep is not None:
            best = best.masked_fill(~d_keep.any(dim=1)[None, None], 0.0)
        if q_keep is not None:
            best = best.masked_fill(~q_keep[i0:i1, :, None], 0.0)
        out[i0:i1] = best.sum(dim=1)
    return out


def maxsim_reference(
    Q: torch.Tensor,
    D: torch.Tensor,
    q_mask: torch.Tensor | None = None,
    d_mask: torch.Tensor | None = None,
    *,
    normalize: bool = False,
) -> torch.Tensor:
    """Dense MaxSim with masks: ``[Nq, Nd]`` (2-D inputs squeeze their dim)."""
    q2, d2 = Q.dim() == 2, D.dim() == 2
    Q3 = Q.unsqueeze(0) if q2 else Q
    D3 = D.unsqueeze(0) if d2 else D
    if Q3.shape[-1] != D3.shape[-1]:
        raise ValueError(f"embedding dims don't match: Q has d={Q3.shape[-1]}, D has d={D3.shape[-1]}")
    Qf, Df = _widen(Q3), _widen(D3)
    if normalize:
        Qf, Df = _unit(Qf), _unit(Df)
    qk = None if q_mask is None else q_mask.bool().reshape(-1, Q3.shape[1]).expand(Q3.shape[0], Q3.shape[1])
    dk = None if d_mask is None else d_mask.bool().reshape(-1, D3.shape[1]).expand(D3.shape[0], D3.shape[1])
    out = _row_max_sum(Qf, Df, qk, dk)
    if q2:
        out = out.squeeze(0)
    if d2:
        out = out.squeeze(-1)
    return out


def plaid_approx_score_reference(
    query_centroid_scores: torch.Tensor,
    codes: torch.Tensor,
    doc_lengths: torch.Tensor,
) -> torch.Tensor:
    """PLAID approximate score: ``sum_s max_{t < len_b} qcs[codes[b, t], s]`` -> ``[B]``."""
    qcs = query_centroid_scores.float()
    B, L = codes.shape
    g = qcs[codes.reshape(-1).long()].view(B, L, -1)
    keep = torch.arange(L, device=codes.device)[None] < doc_lengths.to(codes.device)[:, None]
    m = g.masked_fill(~keep[..., None], NEG_INF).amax(dim=1) if L else torch.full(
        (B, qcs.shape[1]), NEG_INF, device=qcs.device)
    return torch.where(torch.isfinite(m), m, torch.zeros_like(m)).sum(dim=-1)


def unpack_residuals_reference(residuals: torch.Tensor, nbits: int, d: int) -> torch.Tensor:
    """Bucket codes ``[..., d]`` int32: feature f is bits ``(f % (8/nbits)) * nbits``
    upward of byte ``f // (8/nbits)`` (little-endian within the byte)."""
    per = 8 // nbits
    f = torch.arange(d, device=residuals.device)
    b = residuals.to(torch.int32)[..., f // per]
    return (b >> ((f % per) * nbits).to(torch.int32)) & ((1 << nbits) - 1)


def _decode(codes, residuals, centroids, bucket_weights, nbits: int, d: int) -> torch.Tensor:
    w = bucket_weights.float()
    bc = unpack_residuals_reference(residuals, nbits, d).clamp(0, w.numel() - 1).long()
    return centroids.float()[codes.long()] + w[bc]


def maxsim_residual_reference(
    Q: torch.Tensor,
    codes: torch.Tensor,
    residuals: torch.Tensor,
    doc_lengths: torch.Tensor,
    centroids: torch.Tensor,
    bucket_weights: torch.Tensor,
    nbits: int,
    *,
    normalize: bool = True,
) -> torch.Tensor:
    """PLAID decode (``centroids[code] + bucket_weights[bucket]``) then MaxSim,
    padded docs ``codes [B, L]`` with ``doc_lengths [B]`` -> ``[Nq, B]``."""
    Q3 = Q.unsqueeze(0) if Q.dim() == 2 else Q
    emb = _decode(codes, residuals, centroids, bucket_weights, nbits, Q3.shape[-1])
    Qf = Q3.float()
    if normalize:
        emb, Qf = _unit(emb), _unit(Qf)
    L = codes.shape[1]
    keep = torch.arange(L, device=codes.device)[None] < doc_lengths.to(codes.device)[:, None]
    return _row_max_sum(Qf, emb, None, keep)


def maxsim_from_hidden_reference(
    Q: torch.Tensor,
    H_d: torch.Tensor,
    W: torch.Tensor,
    b: torch.Tensor | None = None,
    d_mask: torch.Tensor | None = None,
    *,
    normalize: bool = True,
) -> torch.Tensor:
    """MaxSim of Q against the projected docs ``H_d @ W.T + b`` (fp32; the docs
    normalised when ``normalize``, the queries taken as given)."""
    q2 = Q.dim() == 2
    Dp = torch.nn.functional.linear(H_d.float(), W.float(), None if b is None else b.float())
    if normalize:
        Dp = _unit(Dp)
    if d_mask is not None and d_mask.dim() == 1:
        d_mask = d_mask.unsqueeze(0)
    out = maxsim_reference(Q.unsqueeze(0) if q2 else Q, Dp, d_mask=d_mask)
    return out.squeeze(0) if q2 else out


def _spans(cu: torch.Tensor) -> list[tuple[int, int]]:
    c = cu.to(torch.int64).cpu().tolist()
    return list(zip(c[:-1], c[1:]))


def maxsim_reference_varlen(
    Q: torch.Tensor,
    D: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_d: torch.Tensor,
) -> torch.Tensor:
    """Packed MaxSim: ``Q [total_q, d]``, ``D [total_d, d]`` with cumulative
    offsets -> ``[Nq, Nd]`` fp32; an empty query or doc scores 0."""
    qs, ds = _spans(cu_seqlens_q), _spans(cu_seqlens_d)
    out = torch.zeros(len(qs), len(ds), device=Q.device, dtype=torch.float32)
    Df = D.float()
    for i, (a, b) in enumerate(qs):
        if b <= a:
            continue
        sim = Q[a:b].float() @ Df.T  # [lq, total_d]
        for j, (c, e) in enumerate(ds):
            if e > c:
                out[i, j] = sim[:, c:e].amax(dim=1).sum()
    return out


def maxsim_reference_scatter(
    Q_packed: torch.Tensor,
    D_packed: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_d: torch.Tensor,
    pair_q_idx: torch.Tensor,
    pair_d_idx: torch.Tensor,
) -> torch.Tensor:
    """Pair-list MaxSim over packed Q / D -> ``[num_pairs]`` fp32."""
    qs, ds = _spans(cu_seqlens_q), _spans(cu_seqlens_d)
    out = torch.zeros(pair_q_idx.numel(), device=Q_packed.device, dtype=torch.float32)
    for k, (i, j) in enumerate(zip(pair_q_idx.cpu().tolist(), pair_d_idx.cpu().tolist())):
        (a, b), (c, e) = qs[i], ds[j]
        if b > a and e > c:
            out[k] = (Q_packed[a:b].float() @ D_packed[c:e].float().T).amax(dim=1).sum()
    return out


def maxsim_padded_reference(
    queries: torch.Tensor,
    documents: torch.Tensor,
    query_lengths: torch.Tensor,
    doc_lengths: torch.Tensor,
) -> torch.Tensor:
    """``queries [B, Lq, d]`` against their own candidates ``documents [B, C, Ld, d]``
    with valid prefix lengths -> ``[B, C]`` fp32."""
    B, Lq, _ = queries.shape
    _, C, Ld, _ = documents.shape
    qk = torch.arange(Lq, device=queries.device)[None] < query_lengths.to(queries.device)[:, None]
    dk = torch.arange(Ld, device=queries.device)[None, None] < doc_lengths.to(queries.device)[..., None]
    out = torch.empty(B, C, dtype=torch.float32, device=queries.device)
    for b in range(B):
        out[b] = _row_max_sum(queries[b : b + 1].float(), documents[b].float(), qk[b : b + 1], dk[b],
                              finite_only=False)[0]
    return out


__all__ = [
    "maxsim_reference",
    "plaid_approx_score_reference",
    "unpack_residuals_reference",
    "maxsim_residual_reference",
    "maxsim_from_hidden_reference",
    "maxsim_reference_varlen",
    "maxsim_reference_scatter",
    "maxsim_padded_reference",
]
