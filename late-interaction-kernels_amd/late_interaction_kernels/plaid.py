"""PLAID / ColBERTv2 compressed-index scoring (reference plaid.py).

* :func:`plaid_approx_score` — centroid-only approximate score (IVF prune).
* :func:`maxsim_residual` — padded ``(codes, residuals)`` decode + L2-normalise + MaxSim.
* :func:`maxsim_residual_varlen` — the same on ragged ``cu_seqlens`` buffers
  (the fast-plaid / ColBERTv2 on-disk layout).
* :func:`retrieve_residual_varlen` — chunked decode+MaxSim followed by the
  fused top-k merge, the end-to-end rerank-and-select step.

A token's embedding is ``centroids[code] + bucket_weights[b_f]`` per feature
``f``, where ``b_f`` is the ``nbits``-bit field ``f`` of the packed residual
row, little-endian within each byte (``reference.py:124-139``). Decode,
normalise and MaxSim are one kernel (the decoded tile only lives in LDS), or,
for large query batches, a decode pass followed by the dense MaxSim kernel.
Gradients flow into Q (codes / residuals are integers; centroids and bucket
weights are treated as frozen, as in the reference).
Out-of-range centroid codes are clamped to 0 and bucket codes to the last
bucket, so corrupt indices cannot fault.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._core import assert_max_seqlen_covers
from .topk import topk_update

_CENT_CODE = {torch.bfloat16: _lib.LIK_BF16, torch.float16: _lib.LIK_F16, torch.float32: _lib.LIK_F32}


def _lq_max(d: int) -> int:
    """Query tokens one launch holds in its column block (B-fragment VGPR budget)."""
    return 512 if d <= 128 else 256


def plaid_approx_score(
    query_centroid_scores: torch.Tensor,
    codes: torch.Tensor,
    doc_lengths: torch.Tensor,
) -> torch.Tensor:
    """``out[b] = sum_s max_{t < len_b} qcs[codes[b, t], s]`` -> ``[B]`` fp32 (empty doc -> 0)."""
    if query_centroid_scores.dim() != 2:
        raise ValueError("query_centroid_scores must be [n_centroids, Lq]")
    if codes.dim() != 2:
        raise ValueError("codes must be [B, max_Ld]")
    if doc_lengths.dim() != 1 or doc_lengths.shape[0] != codes.shape[0]:
        raise ValueError("doc_lengths must be [B] with B matching codes")
    _lib.require_gpu(query_centroid_scores, codes, doc_lengths)
    qcs = query_centroid_scores.contiguous().to(torch.float32)
    codes = codes.contiguous().to(torch.int32)
    lens = doc_lengths.contiguous().to(torch.int64)
    n_cent, Lq = qcs.shape
    B, L = codes.shape
    out = torch.empty(B, device=codes.device, dtype=torch.float32)
    if B == 0:
        return out
    lib = _lib.load()
    with torch.cuda.device(codes.device):
        rc = lib.lik_plaid_approx_score(
            qcs.data_ptr(), n_cent, Lq, qcs.stride(0), qcs.stride(1), codes.data_ptr(), B, L,
            codes.stride(0), lens.data_ptr(), out.data_ptr(), _lib.stream_of(out),
        )
    _lib.check(rc, "lik_plaid_approx_score")
    return out


def _check_nbits(nbits: int) -> None:
    if nbits not in (2, 4, 8):
        raise ValueError(f"nbits must be 2, 4, or 8; got {nbits}")


def _prep_q(Q: torch.Tensor) -> torch.Tensor:
    # Compute dtype: fp16 if Q is fp16, else bf16 (reference plaid.py:914).
    Q = Q.to(torch.float16 if Q.dtype == torch.float16 else torch.bfloat16)
    return _lib.prepare_tokens(Q)


def _plaid_launch(Q, docs: _lib.LikPlaidDocs, normalize: bool, out: torch.Tensor) -> None:
    Nq, Lq, d = Q.shape
    lib = _lib.load()
    flags = _lib.LIK_NORMALIZE if normalize else 0
    # Long queries: MaxSim adds over query tokens, so score column-block-sized
    # query slices and sum them.
    step = _lq_max(d)
    starts = list(range(0, Lq, step)) or [0]
    tmp = out if len(starts) == 1 else torch.empty_like(out)
    for n, s0 in enumerate(starts):
        Qc = Q[:, s0 : s0 + step]
        qs = _lib.seqs(Qc, n=Nq, length=Qc.shape[1], stride_n=Qc.stride(0), stride_l=Qc.stride(1))
        dst = out if n == 0 else tmp
        with torch.cuda.device(Q.device):
            rc = lib.lik_plaid_maxsim_ex(
                ctypes.byref(qs), ctypes.byref(docs), flags, dst.data_ptr(), dst.stride(0), dst.stride(1),
                _lib.call_opts(), _lib.stream_of(dst),
            )
        _lib.check(rc, "lik_plaid_maxsim")
        if n > 0:
            out.add_(tmp)


def _plaid_docs(codes, residuals, centroids, bucket_weights, nbits, d, *, cu=None, lengths=None,
                n: int, max_len: int, codes_stride_n: int = 0) -> _lib.LikPlaidDocs:
    p = _lib.LikPlaidDocs()
    p.codes = codes.data_ptr()
    p.residuals = residuals.data_ptr()
    p.cu_seqlens = _lib.ptr(cu)
    p.lengths = _lib.ptr(lengths)
    p.n = n
    p.max_len = max_len
    p.codes_stride_n = codes_stride_n
    p.res_stride_tok = residuals.shape[-1]
    p.centroids = centroids.data_ptr()
    p.centroid_dtype = _CENT_CODE[centroids.dtype]
    p.dim = d
    p.n_centroids = centroids.shape[0]
    p.cent_stride = centroids.stride(0)
    p.bucket_weights = bucket_weights.data_ptr()
    p.n_buckets = bucket_weights.numel()
    p.nbits = nbits
    return p


def _prep_index(residuals, centroids, bucket_weights, nbits, d):
    if d % 8 != 0:
        raise ValueError(f"PLAID scoring needs d % 8 == 0; got d={d}")
    packed_dim = residuals.shape[-1]
    expected = (d * nbits + 7) // 8
    if packed_dim != expected:
        raise ValueError(f"residuals last dim {packed_dim} != expected {expected} for d={d}, nbits={nbits}")
    if centroids.dim() != 2 or centroids.shape[1] != d:
        raise ValueError(f"centroids must be [n_centroids, d={d}]; got {tuple(centroids.shape)}")
    if centroids.dtype not in _CENT_CODE:
        centroids = centroids.to(torch.float32)
    centroids = centroids.contiguous()
    bw = bucket_weights.contiguous().to(torch.float32)
    if not 1 <= bw.numel() <= 256:
        raise ValueError("bucket_weights must hold 1..256 values")
    return residuals.contiguous().to(torch.uint8), centroids, bw


def maxsim_residual(
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
    """Fused PLAID residual decode + L2-normalise + MaxSim on padded docs.

    Args:
        Q: ``[Nq, Lq, d]`` (or ``[Lq, d]``).
        codes: ``[Nd, max_Ld]`` integer centroid codes.
        residuals: ``[Nd, max_Ld, ceil(d*nbits/8)]`` uint8.
        doc_lengths: ``[Nd]`` valid lengths.
        centroids: ``[n_centroids, d]`` fp16/bf16/fp32.
        bucket_weights: ``[2**nbits]`` fp32.
        nbits: 2, 4 or 8.
    Returns:
        ``[Nq, Nd]`` fp32 (``[Nd]`` for 2-D Q). Differentiable in ``Q``.
    """
    _check_nbits(nbits)
    if codes.dim() != 2:
        raise ValueError("codes must be [Nd, max_Ld]")
    if residuals.dim() != 3:
        raise ValueError("residuals must be [Nd, max_Ld, packed_dim]")
    q_squeeze = Q.dim() == 2
    if q_squeeze:
        Q = Q.unsqueeze(0)
    _lib.require_gpu(Q, codes, residuals, doc_lengths, centroids, bucket_weights)
    Nq, Lq, d = Q.shape
    Nd, L = codes.shape
    residuals, centroids, bw = _prep_index(residuals, centroids, bucket_weights, nbits, d)
    if torch.is_grad_enabled() and Q.requires_grad and Nq and Nd and Lq and L:
        lens = doc_lengths.contiguous().to(torch.int32)
        out = _residual_with_q_grad(Q, codes.reshape(-1), residuals.reshape(Nd * L, -1), centroids, bw, nbits,
                                    lengths=lens, Nd=Nd, L=L, normalize=normalize)
        return out.squeeze(0) if q_squeeze else out
    out = torch.empty(Nq, Nd, device=Q.device, dtype=torch.float32)
    if Nq and Nd:
        if Lq == 0 or L == 0:
            out.zero_()
        else:
            codes = codes.contiguous().to(torch.int32)
            lens = doc_lengths.contiguous().to(torch.int32)
            docs = _plaid_docs(codes, residuals, centroids, bw, nbits, d, lengths=lens, n=Nd, max_len=L,
                               codes_stride_n=L)
            _plaid_launch(_prep_q(Q), docs, normalize, out)
    return out.squeeze(0) if q_squeeze else out


def maxsim_residual_varlen(
    Q: torch.Tensor,
    codes_flat: torch.Tensor,
    residuals_flat: torch.Tensor,
    cu_seqlens_d: torch.Tensor,
    centroids: torch.Tensor,
    bucket_weights: torch.Tensor,
    nbits: int,
    *,
    max_seqlen_d: int | None = None,
    normalize: bool = True,
) -> torch.Tensor:
    """Ragged PLAID decode + MaxSim on ``cu_seqlens``-indexed flat buffers.

    ``max_seqlen_d`` is accepted for API compatibility (checked on device if
    given); the kernel does not need it, so no device->host sync happens.
    Returns ``[Nq, Nd]`` fp32 (``[Nd]`` for 2-D Q); an empty doc scores 0.
    """
    _check_nbits(nbits)
    q_squeeze = Q.dim() == 2
    if q_squeeze:
        Q = Q.unsqueeze(0)
    if codes_flat.dim() != 1:
        raise ValueError("codes_flat must be 1-D [total_d_tokens]")
    if residuals_flat.dim() != 2:
        raise ValueError("residuals_flat must be 2-D [total_d_tokens, packed_dim]")
    if cu_seqlens_d.dim() != 1:
        raise ValueError("cu_seqlens_d must be 1-D [Nd + 1]")
    _lib.require_gpu(Q, codes_flat, residuals_flat, cu_seqlens_d, centroids, bucket_weights)
    Nq, Lq, d = Q.shape
    residuals_flat, centroids, bw = _prep_index(residuals_flat, centroids, bucket_weights, nbits, d)
    cu = cu_seqlens_d.contiguous().to(torch.int32)
    Nd = cu.numel() - 1
    if max_seqlen_d is not None:
        assert_max_seqlen_covers(cu, int(max_seqlen_d), "max_seqlen_d")
    if torch.is_grad_enabled() and Q.requires_grad and Nq and Nd > 0 and Lq and codes_flat.numel():
        out = _residual_with_q_grad(Q, codes_flat, residuals_flat, centroids, bw, nbits, cu=cu, Nd=Nd, L=0,
                                    normalize=normalize)
        return out.squeeze(0) if q_squeeze else out
    out = torch.empty(Nq, max(Nd, 0), device=Q.device, dtype=torch.float32)
    if Nq and Nd > 0:
        if Lq == 0 or codes_flat.numel() == 0:
            out.zero_()
        else:
            codes = codes_flat.contiguous().to(torch.int32)
            docs = _plaid_docs(codes, residuals_flat, centroids, bw, nbits, d, cu=cu, n=Nd,
                               max_len=int(max_seqlen_d or 0))
            Qp = _prep_q(Q)
            if _use_decode_route(Nq, Lq):
                cu_host = cu.cpu()  # the route's one device->host sync: chunk token bounds
                buf = None
                for j0, j1 in _token_chunks(cu_host, 0, Nd):
                    buf = _decoded_chunk_scores(Qp, docs, cu, j0, j1, int(cu_host[j0]), int(cu_host[j1]),
                                                normalize, out[:, j0:j1], buf)
            else:
                _plaid_launch(Qp, docs, normalize, out)
    return out.squeeze(0) if q_squeeze else out


# Decode-once route. The fused kernel decodes each document once per
# 512-token query block (column group); with many query tokens that repeats
# the decode work, so above this size each doc chunk is decoded once into
# HBM (lik_plaid_decode) and scored by the dense MaxSim kernel. Both routes
# produce bitwise the same bf16/fp16 rows and the same scores.
_DECODE_ROUTE_MIN_QTOK = 2048
_DECODE_TOKENS = 1 << 20  # tokens decoded per chunk (256 MB of bf16 rows at d = 128)


def _token_chunks(cu_host: torch.Tensor, j0: int, j1: int):
    """Split docs [j0, j1) into consecutive ranges of at most _DECODE_TOKENS
    tokens each (a longer single doc forms its own range)."""
    while j0 < j1:
        t0 = int(cu_host[j0])
        e = int(torch.searchsorted(cu_host, t0 + _DECODE_TOKENS, right=True)) - 1
        e = min(max(e, j0 + 1), j1)
        yield j0, e
        j0 = e


def _use_decode_route(Nq: int, Lq: int) -> bool:
    """``_lib.launch_options(plaid_route="fused" | "decode")`` forces a route;
    otherwise by query-token count."""
    forced = _lib.plaid_route()
    if forced == "fused":
        return False
    if forced == "decode":
        return True
    return Nq * Lq >= _DECODE_ROUTE_MIN_QTOK


def decode_residual_tokens(
    codes_flat: torch.Tensor,
    residuals_flat: torch.Tensor,
    centroids: torch.Tensor,
    bucket_weights: torch.Tensor,
    nbits: int,
    *,
    normalize: bool = True,
    dtype: torch.dtype = torch.bfloat16,
) -> torch.Tensor:
    """Decode PLAID tokens to ``[T, d]`` rows: ``centroids[code] + bucket_weights[field]``
    per feature (little-endian fields, reference.py:124-139, 164-167), L2-normalised
    when ``normalize``, rounded once to ``dtype`` (bf16 or fp16)."""
    _check_nbits(nbits)
    if codes_flat.dim() != 1 or residuals_flat.dim() != 2 or residuals_flat.shape[0] != codes_flat.shape[0]:
        raise ValueError("codes_flat must be [T] and residuals_flat [T, packed_dim]")
    if dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("dtype must be torch.bfloat16 or torch.float16")
    _lib.require_gpu(codes_flat, residuals_flat, centroids, bucket_weights)
    d = centroids.shape[-1]
    residuals_flat, centroids, bw = _prep_index(residuals_flat, centroids, bucket_weights, nbits, d)
    codes = codes_flat.contiguous().to(torch.int32)
    T = codes.shape[0]
    out = torch.empty(T, d, device=codes.device, dtype=dtype)
    if T:
        docs = _plaid_docs(codes, residuals_flat, centroids, bw, nbits, d, n=0, max_len=0)
        _decode_into(docs, 0, T, normalize, out)
    return out


class _ResidualQGradFn(torch.autograd.Function):
    """PLAID MaxSim differentiable in Q only (reference plaid.py:518-616): codes and
    residuals are integers, centroids / bucket weights frozen. Forward decodes the
    docs once (lik_plaid_decode) and runs the argmax-saving MaxSim on the decoded
    rows; backward runs the grad_Q kernel against the same rows."""

    @staticmethod
    def forward(ctx, Q, docs_tuple, cu, lengths, Nd, L, normalize):
        codes, residuals, centroids, bw, nbits = docs_tuple
        Qp = _lib.prepare_tokens(Q.detach())
        Nq, Lq, d = Qp.shape
        T = codes.shape[0]
        docs = _plaid_docs(codes, residuals, centroids, bw, nbits, d, n=0, max_len=0)
        dec = torch.empty(max(T, 1), d, device=Q.device, dtype=Qp.dtype)
        if T:
            _decode_into(docs, 0, T, normalize, dec)
        qs = _lib.seqs(Qp, n=Nq, length=Lq, stride_n=Qp.stride(0), stride_l=Qp.stride(1))
        if cu is not None:
            ds = _lib.seqs(dec, n=Nd, length=0, stride_l=dec.stride(0), cu=cu)
        else:
            ds = _lib.seqs(dec, n=Nd, length=L, stride_n=L * dec.stride(0), stride_l=dec.stride(0), lengths=lengths)
        flags = _lib.LIK_NORMALIZE_Q if normalize else 0
        out = torch.empty(Nq, Nd, device=Q.device, dtype=torch.float32)
        argmax = torch.full((Nq * Nd, Lq), -1, device=Q.device, dtype=torch.int32)
        lib = _lib.load()
        nbytes = lib.lik_maxsim_workspace_size(ctypes.byref(qs), ctypes.byref(ds), flags)
        ws = _lib.workspace(nbytes, Q.device)
        with torch.cuda.device(Q.device):
            rc = lib.lik_maxsim_argmax(ctypes.byref(qs), ctypes.byref(ds), flags, out.data_ptr(), out.stride(0),
                                       out.stride(1), argmax.data_ptr(), _lib.ptr(ws), nbytes, _lib.stream_of(out))
        _lib.check(rc, "lik_maxsim_argmax")
        ctx.save_for_backward(Qp, dec, argmax, cu, lengths)
        ctx.meta = (Nd, L, normalize, Q.shape[-1], Q.dtype)
        ctx.mark_non_differentiable(argmax)
        return out

    @staticmethod
    def backward(ctx, grad_scores):
        Qp, dec, argmax, cu, lengths = ctx.saved_tensors
        Nd, L, normalize, d_in, qdt = ctx.meta
        Nq, Lq, d = Qp.shape
        g = grad_scores.to(torch.float32).contiguous()
        qs = _lib.seqs(Qp, n=Nq, length=Lq, stride_n=Qp.stride(0), stride_l=Qp.stride(1))
        if cu is not None:
            ds = _lib.seqs(dec, n=Nd, length=0, stride_l=dec.stride(0), cu=cu)
        else:
            ds = _lib.seqs(dec, n=Nd, length=L, stride_n=L * dec.stride(0), stride_l=dec.stride(0), lengths=lengths)
        flags = _lib.LIK_NORMALIZE_Q if normalize else 0
        gq = torch.empty_like(Qp)
        lib = _lib.load()
        nbytes = lib.lik_maxsim_backward_workspace_size(ctypes.byref(qs), ctypes.byref(ds), flags)
        ws = _lib.workspace(nbytes, Qp.device)
        with torch.cuda.device(Qp.device):
            rc = lib.lik_maxsim_backward(g.data_ptr(), g.stride(0), ctypes.byref(qs), ctypes.byref(ds),
                                         argmax.data_ptr(), flags, gq.data_ptr(), None, _lib.ptr(ws), nbytes,
                                         _lib.stream_of(gq))
        _lib.check(rc, "lik_maxsim_backward")
        return gq[..., :d_in].to(qdt), None, None, None, None, None, None


def _residual_with_q_grad(Q, codes_flat, residuals, centroids, bw, nbits, *, cu=None, lengths=None, Nd, L,
                          normalize):
    Qc = Q.to(torch.float16 if Q.dtype == torch.float16 else torch.bfloat16)  # differentiable cast
    codes = codes_flat.contiguous().to(torch.int32)
    return _ResidualQGradFn.apply(Qc, (codes, residuals, centroids, bw, nbits), cu, lengths, Nd, L, normalize)


def _decode_into(docs: _lib.LikPlaidDocs, t0: int, t1: int, normalize: bool, out: torch.Tensor) -> None:
    lib = _lib.load()
    with torch.cuda.device(out.device):
        rc = lib.lik_plaid_decode(
            ctypes.byref(docs), t0, t1, _lib.LIK_NORMALIZE if normalize else 0, _lib.DTYPE_CODE[out.dtype],
            out.data_ptr(), out.stride(0), _lib.stream_of(out),
        )
    _lib.check(rc, "lik_plaid_decode")


def _decoded_chunk_scores(Qp, docs, cu, j0: int, j1: int, t0: int, t1: int, normalize: bool,
                          out: torch.Tensor, buf: torch.Tensor | None) -> torch.Tensor:
    """Scores of docs [j0, j1) (tokens [t0, t1)) into ``out`` ([Nq, j1-j0] view):
    decode the chunk once, then dense packed MaxSim with query-only normalise.
    Returns the decode buffer for reuse."""
    d = Qp.shape[-1]
    ntok = t1 - t0
    if buf is None or buf.shape[0] < ntok or buf.dtype != Qp.dtype:
        buf = torch.empty(max(ntok, 1), d, device=Qp.device, dtype=Qp.dtype)
    if ntok == 0:
        out.zero_()
        return buf
    _decode_into(docs, t0, t1, normalize, buf)
    cu_rel = cu[j0 : j1 + 1] - t0
    Nq, Lq, _ = Qp.shape
    qs = _lib.seqs(Qp, n=Nq, length=Lq, stride_n=Qp.stride(0), stride_l=Qp.stride(1))
    ds = _lib.seqs(buf, n=j1 - j0, length=0, stride_l=buf.stride(0), cu=cu_rel)
    flags = _lib.LIK_NORMALIZE_Q if normalize else 0
    lib = _lib.load()
    opts = _lib.call_opts()
    nbytes = lib.lik_maxsim_workspace_size_ex(ctypes.byref(qs), ctypes.byref(ds), flags, opts)
    ws = _lib.workspace(nbytes, Qp.device)
    with torch.cuda.device(Qp.device):
        rc = lib.lik_maxsim_ex(ctypes.byref(qs), ctypes.byref(ds), flags, 1.0, out.data_ptr(), out.stride(0),
                               out.stride(1), _lib.ptr(ws), nbytes, opts, _lib.stream_of(out))
    _lib.check(rc, "lik_maxsim")
    return buf


def retrieve_residual_varlen(
    Q: torch.Tensor,
    codes_flat: torch.Tensor,
    residuals_flat: torch.Tensor,
    cu_seqlens_d: torch.Tensor,
    centroids: torch.Tensor,
    bucket_weights: torch.Tensor,
    nbits: int,
    top_k: int,
    *,
    chunk: int | None = 4096,
    normalize: bool = True,
    largest: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-``top_k`` documents of a PLAID-compressed corpus per query.

    Scores ``chunk`` documents at a time with :func:`maxsim_residual_varlen`
    and folds each ``[Nq, chunk]`` block into the running top-k with the fused
    merge (``retrieve``'s chunk semantics, ties to the lower doc index).
    Returns ``(scores [Nq, k], indices [Nq, k])`` with ``k = min(top_k, Nd)``.
    """
    if top_k <= 0:
        raise ValueError(f"top_k must be positive, got {top_k}")
    q_squeeze = Q.dim() == 2
    if q_squeeze:
        Q = Q.unsqueeze(0)
    cu = cu_seqlens_d.contiguous().to(torch.int32)
    Nd = cu.numel() - 1
    k = min(top_k, max(Nd, 0))
    Nq = Q.shape[0]
    if k == 0:
        e = torch.empty(Nq, 0, device=Q.device)
        return (e[0], e.long()[0]) if q_squeeze else (e, e.long())
    cs = Nd if chunk is None or chunk >= Nd else int(chunk)
    if cs <= 0:
        raise ValueError(f"chunk must be positive, got {chunk}")
    run_s = run_i = None
    with torch.no_grad():
        if _use_decode_route(Nq, Q.shape[1]) and Q.shape[1] > 0:
            # decode-once route: one sync for the chunks' token bounds, one
            # decode buffer reused by every chunk
            _check_nbits(nbits)
            _lib.require_gpu(Q, codes_flat, residuals_flat, cu_seqlens_d, centroids, bucket_weights)
            d = Q.shape[-1]
            res, cent, bw = _prep_index(residuals_flat, centroids, bucket_weights, nbits, d)
            codes = codes_flat.contiguous().to(torch.int32)
            docs = _plaid_docs(codes, res, cent, bw, nbits, d, cu=cu, n=Nd, max_len=0)
            Qp = _prep_q(Q)
            cu_host = cu.cpu()  # the route's one device->host sync: decode chunk bounds
            buf = None
            scores = torch.empty(Nq, cs, device=Q.device, dtype=torch.float32)
            for start in range(0, Nd, cs):
                end = min(start + cs, Nd)
                s = scores[:, : end - start]
                for j0, j1 in _token_chunks(cu_host, start, end):
                    buf = _decoded_chunk_scores(Qp, docs, cu, j0, j1, int(cu_host[j0]), int(cu_host[j1]), normalize,
                                                s[:, j0 - start : j1 - start], buf)
                run_s, run_i = topk_update(s, start, run_s, run_i, k, largest)
        else:
            for start in range(0, Nd, cs):
                end = min(start + cs, Nd)
                s = maxsim_residual_varlen(Q, codes_flat, residuals_flat, cu[start : end + 1], centroids,
                                           bucket_weights, nbits, normalize=normalize)
                run_s, run_i = topk_update(s, start, run_s, run_i, k, largest)
    if q_squeeze:
        return run_s[0], run_i[0]
    return run_s, run_i


class ResidualIndex:
    """A PLAID-compressed corpus prepared once for repeated few-query scoring.

    Same inputs as :func:`maxsim_residual_varlen` (``codes_flat``,
    ``residuals_flat``, ``cu_seqlens_d``, ``centroids``, ``bucket_weights``,
    ``nbits``). Construction computes every token's inverse L2 norm once and
    stores it beside the token's code (``lik_plaid_token_records``: an
    8-byte (code, norm) record per token, one decode pass). Scoring up to 64
    queries of at most 32 tokens then runs ``lik_plaid_maxsim_qc``: per query
    a table of query-centroid scores (``[n_centroids, 32]`` fp16), and a scan
    that reads each token's record and residual bytes from HBM and one 64-byte
    table row instead of a 256-byte centroid row. Scores
    match :func:`maxsim_residual_varlen` within bf16 rounding (the centroid
    term is rounded to fp16). Larger batches, queries needing gradients,
    layouts the scan cannot take, and query / centroid norms whose products
    could leave fp16's range use :func:`maxsim_residual_varlen`.

    The tensors are borrowed: modifying them after construction invalidates
    the precomputed norms.
    """

    def __init__(self, codes_flat, residuals_flat, cu_seqlens_d, centroids, bucket_weights, nbits: int):
        _check_nbits(nbits)
        if codes_flat.dim() != 1 or residuals_flat.dim() != 2 or cu_seqlens_d.dim() != 1:
            raise ValueError("codes_flat [T], residuals_flat [T, packed_dim] and cu_seqlens_d [Nd + 1] expected")
        _lib.require_gpu(codes_flat, residuals_flat, cu_seqlens_d, centroids, bucket_weights)
        d = centroids.shape[-1]
        self.residuals, self.centroids, self.bucket_weights = _prep_index(residuals_flat, centroids, bucket_weights,
                                                                          nbits, d)
        self.codes = codes_flat.contiguous().to(torch.int32)
        self.cu = cu_seqlens_d.contiguous().to(torch.int32)
        self.nbits = nbits
        self.d = d
        self.n_docs = self.cu.numel() - 1
        T = self.codes.numel()
        # largest centroid norm (one sync, here): bounds |q.c| for the fp16 table
        self._cent_norm_max = float(self.centroids.float().norm(dim=-1).max()) if self.centroids.shape[0] else 0.0
        # (code, inverse norm) per token, as int32 pairs
        self.token_rec = torch.empty(T, 2, device=self.codes.device, dtype=torch.int32)
        if T:
            docs = self._docs()
            lib = _lib.load()
            with torch.cuda.device(self.codes.device):
                rc = lib.lik_plaid_token_records(ctypes.byref(docs), 0, T, self.token_rec.data_ptr(),
                                                 _lib.stream_of(self.token_rec))
            _lib.check(rc, "lik_plaid_token_records")

    @property
    def token_inv(self) -> torch.Tensor:
        """``[T]`` fp32 inverse norms of the tokens: a strided view of the
        records (C-ABI callers pass ``token_rec`` with ``LIK_TOKEN_RECORDS``,
        or a contiguous copy of this view without it)."""
        return self.token_rec[:, 1].view(torch.float32)

    def _docs(self) -> _lib.LikPlaidDocs:
        return _plaid_docs(self.codes, self.residuals, self.centroids, self.bucket_weights, self.nbits, self.d,
                           cu=self.cu, n=self.n_docs, max_len=0)

    def _scan_ok(self, Qp: torch.Tensor) -> bool:
        Nq, Lq, d = Qp.shape
        return (Nq <= 64 and 0 < Lq <= 32 and d <= 128 and self.centroids.dtype == Qp.dtype
                and self.residuals.shape[-1] % 16 == 0 and self.residuals.data_ptr() % 16 == 0)

    # the scan keeps q.c in an fp16 table: beyond this bound the call takes
    # maxsim_residual_varlen (fp16's largest finite value is 65504)
    _TABLE_BOUND = 6.0e4

    def _table_fits(self, Qp: torch.Tensor, normalize: bool) -> bool:
        """|q.c| <= |q| max|c| stays below the fp16 bound. With normalize the
        query rows are unit rows (no sync); without, the largest query-token
        norm is read back (one sync per call). A NaN bound (NaN inputs) passes:
        the scan propagates NaN like the other routes."""
        qmax = 1.0 if normalize else float(Qp.float().norm(dim=-1).max()) if Qp.numel() else 0.0
        return not (qmax * self._cent_norm_max >= self._TABLE_BOUND)

    def score(self, Q: torch.Tensor, *, normalize: bool = True) -> torch.Tensor:
        """``[Nq, Nd]`` fp32 scores (``[Nd]`` for 2-D Q), as :func:`maxsim_residual_varlen`."""
        q_squeeze = Q.dim() == 2
        if q_squeeze:
            Q = Q.unsqueeze(0)
        if Q.shape[-1] != self.d:
            raise ValueError(f"Q has d={Q.shape[-1]}, the index d={self.d}")
        _lib.require_gpu(Q)
        Qp = _prep_q(Q)
        if (torch.is_grad_enabled() and Q.requires_grad) or not self._scan_ok(Qp) or not self._table_fits(Qp, normalize):
            out = maxsim_residual_varlen(Q, self.codes, self.residuals, self.cu, self.centroids, self.bucket_weights,
                                         self.nbits, normalize=normalize)
            return out.squeeze(0) if q_squeeze else out
        Nq, Lq, _ = Qp.shape
        out = torch.empty(Nq, max(self.n_docs, 0), device=Q.device, dtype=torch.float32)
        if Nq and self.n_docs > 0:
            if self.codes.numel() == 0:
                return out.zero_()
            docs = self._docs()
            qs = _lib.seqs(Qp, n=Nq, length=Lq, stride_n=Qp.stride(0), stride_l=Qp.stride(1))
            lib = _lib.load()
            nbytes = lib.lik_plaid_maxsim_qc_workspace_size(ctypes.byref(qs), ctypes.byref(docs))
            ws = _lib.workspace(nbytes, Q.device)
            flags = (_lib.LIK_NORMALIZE if normalize else 0) | _lib.LIK_TOKEN_RECORDS
            with torch.cuda.device(Q.device):
                rc = lib.lik_plaid_maxsim_qc(ctypes.byref(qs), ctypes.byref(docs), self.token_rec.data_ptr(), flags,
                                             out.data_ptr(), out.stride(0), out.stride(1), _lib.ptr(ws), nbytes,
                                             _lib.call_opts(), _lib.stream_of(out))
            _lib.check(rc, "lik_plaid_maxsim_qc")
        return out.squeeze(0) if q_squeeze else out

    def retrieve(self, Q: torch.Tensor, top_k: int, *, chunk: int | None = None, normalize: bool = True,
                 largest: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
        """Top-``top_k`` documents per query, as :func:`retrieve_residual_varlen`
        (ties to the lower doc index). The few-query scan scores every document
        in one launch (``chunk`` does not change the result, only how the
        fallback route bounds its score buffers)."""
        if top_k <= 0:
            raise ValueError(f"top_k must be positive, got {top_k}")
        q_squeeze = Q.dim() == 2
        Q3 = Q.unsqueeze(0) if q_squeeze else Q
        if not self._scan_ok(_prep_q(Q3)) or (torch.is_grad_enabled() and Q.requires_grad):
            return retrieve_residual_varlen(Q, self.codes, self.residuals, self.cu, self.centroids,
                                            self.bucket_weights, self.nbits, top_k, chunk=chunk, normalize=normalize,
                                            largest=largest)
        k = min(top_k, max(self.n_docs, 0))
        Nq = Q3.shape[0]
        if k == 0:
            e = torch.empty(Nq, 0, device=Q.device)
            return (e[0], e.long()[0]) if q_squeeze else (e, e.long())
        with torch.no_grad():
            s = self.score(Q3, normalize=normalize)
            run_s, run_i = topk_update(s, 0, None, None, k, largest)
        return (run_s[0], run_i[0]) if q_squeeze else (run_s, run_i)


__all__ = [
    "ResidualIndex",
    "decode_residual_tokens",
    "plaid_approx_score",
    "maxsim_residual",
    "maxsim_residual_varlen",
    "retrieve_residual_varlen",
]
