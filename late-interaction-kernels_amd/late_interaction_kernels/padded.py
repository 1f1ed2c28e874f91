"""Padded reranking inputs (reference padded.py).

``maxsim_padded`` scores ``[B, Lq, d]`` queries against ``[B, C, Ld, d]``
candidates with per-row valid lengths. The reference packs the valid tokens
(``pack_padded``) and runs a pair-list kernel; here the padded tensors go to
the KD-layout kernel directly with the lengths as prefix bounds, so no
packing copy and no device->host sync happen. ``pack_padded`` is kept as a
public helper producing the same ``PackedBatch`` as the reference.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ._core import dense_maxsim, unify_dtype
from .autograd import _needs_grad, _score


@dataclass(frozen=True)
class PackedBatch:
    """Result of :func:`pack_padded` (field order as in the reference)."""

    Q_packed: torch.Tensor
    cu_seqlens_q: torch.Tensor
    D_packed: torch.Tensor
    cu_seqlens_d: torch.Tensor
    pair_q_idx: torch.Tensor
    pair_d_idx: torch.Tensor
    max_seqlen_q: int
    max_seqlen_d: int

    def __iter__(self):
        yield self.Q_packed
        yield self.cu_seqlens_q
        yield self.D_packed
        yield self.cu_seqlens_d
        yield self.pair_q_idx
        yield self.pair_d_idx
        yield self.max_seqlen_q
        yield self.max_seqlen_d


def _check_padded(queries, documents, query_lengths, doc_lengths):
    if queries.dim() != 3:
        raise ValueError(f"queries must be [B, Lq, d]; got shape {tuple(queries.shape)}")
    if documents.dim() != 4:
        raise ValueError(f"documents must be [B, C, Ld, d]; got shape {tuple(documents.shape)}")
    B, _, d = queries.shape
    Bd, C, _, Dd = documents.shape
    if B != Bd:
        raise ValueError(f"batch size mismatch: queries B={B}, documents B={Bd}")
    if d != Dd:
        raise ValueError(f"embedding dim mismatch: queries d={d}, documents d={Dd}")
    if tuple(query_lengths.shape) != (B,):
        raise ValueError(f"query_lengths must be [B={B}]; got {tuple(query_lengths.shape)}")
    if tuple(doc_lengths.shape) != (B, C):
        raise ValueError(f"doc_lengths must be [B={B}, C={C}]; got {tuple(doc_lengths.shape)}")


def pack_padded(
    queries: torch.Tensor,
    documents: torch.Tensor,
    query_lengths: torch.Tensor,
    doc_lengths: torch.Tensor,
    *,
    validate: bool = False,
) -> PackedBatch:
    """Convert padded reranking tensors to the packed (cu_seqlens) layout.

    Row-major over ``(b, c)``: ``pair_q_idx[b*C + c] = b``, ``pair_d_idx[b*C + c] = b*C + c``.
    One device->host sync fetches both maxima.
    """
    _check_padded(queries, documents, query_lengths, doc_lengths)
    B, Lq_max, d = queries.shape
    _, C, Ld_max, _ = documents.shape
    device = queries.device
    if B == 0:
        z = torch.zeros(1, dtype=torch.int32, device=device)
        e = torch.zeros(0, dtype=torch.int32, device=device)
        return PackedBatch(queries.reshape(0, d), z, documents.reshape(0, d), z.clone(), e, e.clone(), 0, 0)
    qlen = query_lengths.to(device=device, dtype=torch.int32)
    dlen = doc_lengths.to(device=device, dtype=torch.int32)
    torch._assert_async(qlen.le(Lq_max).all())
    torch._assert_async(dlen.le(Ld_max).all())
    if validate:
        if bool((qlen <= 0).any()):
            raise ValueError("query_lengths must all be > 0")
        if bool((dlen <= 0).any()):
            raise ValueError("doc_lengths must all be > 0")
        if bool((qlen > Lq_max).any()) or bool((dlen > Ld_max).any()):
            raise ValueError("a length exceeds the padded extent")
    q_keep = torch.arange(Lq_max, device=device, dtype=torch.int32)[None, :] < qlen[:, None]
    Q_packed = queries.reshape(B * Lq_max, d)[q_keep.reshape(-1)]
    d_keep = torch.arange(Ld_max, device=device, dtype=torch.int32)[None, None, :] < dlen[:, :, None]
    D_packed = documents.reshape(B * C * Ld_max, d)[d_keep.reshape(-1)]
    cu_q = torch.zeros(B + 1, dtype=torch.int32, device=device)
    cu_q[1:] = qlen.cumsum(0)
    cu_d = torch.zeros(B * C + 1, dtype=torch.int32, device=device)
    cu_d[1:] = dlen.reshape(-1).cumsum(0)
    flat = torch.arange(B * C, dtype=torch.int32, device=device)
    max_q, max_d = torch.stack([qlen.max(), dlen.max()]).tolist()
    return PackedBatch(Q_packed, cu_q, D_packed, cu_d, (flat // C).contiguous(), flat, int(max_q), int(max_d))


def maxsim_padded(
    queries: torch.Tensor,
    documents: torch.Tensor,
    query_lengths: torch.Tensor,
    doc_lengths: torch.Tensor,
    *,
    validate: bool = False,
) -> torch.Tensor:
    """Score ``C`` candidates per query from padded inputs -> ``[B, C]`` fp32.

    Tokens at positions ``>= length`` are ignored; a zero-length query or
    document scores 0 (``reference.py:272-306``). Lengths above the padded
    extent are clamped to it (``validate=True`` raises instead).
    """
    _check_padded(queries, documents, query_lengths, doc_lengths)
    B, Lq, d = queries.shape
    _, C, Ld, _ = documents.shape
    if validate:
        ql = query_lengths
        dl = doc_lengths
        if bool((ql <= 0).any()) or bool((dl <= 0).any()):
            raise ValueError("lengths must all be > 0")
        if bool((ql > Lq).any()) or bool((dl > Ld).any()):
            raise ValueError("a length exceeds the padded extent")
    Q, D = unify_dtype(queries, documents)
    if B == 0 or C == 0:
        return torch.zeros(B, C, device=queries.device, dtype=torch.float32)
    if _needs_grad(queries, documents):
        # training: the KD layout with length masks through the argmax forward
        # and the deterministic backward (the reference's pair-list backward,
        # score_pairs.py:344-420, computes the same gradients)
        dev = queries.device
        qm = torch.arange(Lq, device=dev)[None, :] < query_lengths.to(dev).reshape(B, 1)
        dm = torch.arange(Ld, device=dev)[None, :] < doc_lengths.to(dev).reshape(B * C, 1)
        return _score(Q, D.reshape(B * C, Ld, d), qm, dm, normalize=False, kd=True)
    return dense_maxsim(
        Q,
        D.reshape(B * C, Ld, d),
        kd=True,
        q_lengths=query_lengths.to(queries.device),
        d_lengths=doc_lengths.reshape(B * C).to(queries.device),
    )


__all__ = ["PackedBatch", "pack_padded", "maxsim_padded"]
