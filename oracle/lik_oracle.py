"""CPU oracle for the MaxSim hot path — TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference library's ground truth
(late_interaction_kernels/reference.py, fp8.py quantisers, topk.py /
retrieve.py chunk merge). Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it, and only as the checker (or, for the CPU
baseline, as the thing timed on the host). The product package never
imports it and has no CPU fallback.

Arithmetic is float64 unless a function says otherwise, so the oracle is at
least as accurate as the reference's fp32 einsum.

Pinning (how each function is checked, see tests/test_oracle.py):
  maxsim / maxsim_kd / maxsim_varlen / maxsim_pairs / maxsim_padded
      - brute-force triple loops on tiny inputs (reference test pattern
        tests/test_reference_cpu.py:117-145), closed forms (Q row == D row
        after normalise -> 1; orthogonal -> 0; all-masked -> 0), and
        cross-identities (varlen == padded, pairs == kd == per-query loop).
  unpack_residuals / pack_residuals
      - exact integer round trip (tests/test_reference_cpu.py:55-72) and
        hand-computed bytes.
  maxsim_residual(_varlen)
      - identity buckets reduce to dense MaxSim over centroids[codes]
        (tests/test_reference_cpu.py:81-104); decode checked on hand bytes.
  quantize_fp8_* / e4m3_round
      - against torch's float8_e4m3fn cast (a library RNE routine) over all
        finite e4m3 values, midpoints and saturation.
  topk_stable / retrieve_chunked
      - against Python's sorted() with key (-score, index); chunked ==
        unchunked (tests/test_retrieve_cpu.py:191-231).
  plaid_approx_score
      - brute force loop, empty docs -> 0, padding invariance
        (tests/test_reference_cpu.py:25-47).
  pack_residuals_colbert / reverse_bits_bytes
      - reversing the bits of every byte of the ColBERT / fast-plaid encoding
        gives exactly pack_residuals (our little-endian layout); hand bytes.
  maxsim_argmax / maxsim_grads
      - argmax against a pure-Python scan (first index of the max, -1 for an
        all-masked doc); gradients against central finite differences of
        maxsim() (away from ties) with and without normalise, masks, KD.
"""

from __future__ import annotations

import numpy as np

NEG_INF = -np.inf


# --------------------------------------------------------------------------- #
# dense MaxSim                                                                #
# --------------------------------------------------------------------------- #


def _normalize(x: np.ndarray) -> np.ndarray:
    """F.normalize(p=2, dim=-1, eps=1e-12): x / max(||x||, 1e-12) (reference.py:73-74)."""
    n = np.sqrt((x * x).sum(-1, keepdims=True))
    return x / np.maximum(n, 1e-12)


def maxsim(Q, D, q_mask=None, d_mask=None, *, normalize=False, dtype=np.float64, q_chunk=64):
    """score[i, j] = sum_{s: q_mask} max_{t: d_mask} <Q[i,s], D[j,t]>  (reference.py:26-98).

    Q [Nq, Lq, d] or [Lq, d]; D [Nd, Ld, d] or [Ld, d]; masks bool [N, L] or [L].
    A row whose max is over no token (or is non-finite) contributes 0
    (reference.py:82-85); masked query tokens contribute 0 (reference.py:87-91).
    2-D inputs squeeze the matching output dim.
    """
    Q = np.asarray(Q, dtype=dtype)
    D = np.asarray(D, dtype=dtype)
    q2, d2 = Q.ndim == 2, D.ndim == 2
    if q2:
        Q = Q[None]
    if d2:
        D = D[None]
    if Q.shape[-1] != D.shape[-1]:
        raise ValueError("embedding dims don't match")
    if normalize:
        Q = _normalize(Q)
        D = _normalize(D)
    Nq, Lq, d = Q.shape
    Nd, Ld, _ = D.shape
    dm = None
    if d_mask is not None:
        dm = np.asarray(d_mask, dtype=bool)
        if dm.ndim == 1:
            dm = dm[None]
        dm = np.broadcast_to(dm, (Nd, Ld))
    qm = None
    if q_mask is not None:
        qm = np.asarray(q_mask, dtype=bool)
        if qm.ndim == 1:
            qm = qm[None]
        qm = np.broadcast_to(qm, (Nq, Lq))
    Df = D.reshape(Nd * Ld, d)
    out = np.zeros((Nq, Nd), dtype=dtype)
    for i0 in range(0, Nq, q_chunk):
        i1 = min(i0 + q_chunk, Nq)
        S = (Q[i0:i1].reshape(-1, d) @ Df.T).reshape(i1 - i0, Lq, Nd, Ld)
        if dm is not None:
            S = np.where(dm[None, None, :, :], S, NEG_INF)
        m = S.max(axis=-1) if Ld > 0 else np.full((i1 - i0, Lq, Nd), NEG_INF)
        m = np.where(np.isfinite(m), m, 0.0)
        if qm is not None:
            m = m * qm[i0:i1, :, None]
        out[i0:i1] = m.sum(axis=1)
    if q2 and d2:
        return out.reshape(())
    if q2:
        return out[0]
    if d2:
        return out[:, 0]
    return out


def maxsim_argmax(Q, D, d_mask=None, *, normalize=False, kd=False):
    """Winner doc-token index per (query i, doc j, query token s) -> int [Nq * docs, Lq]
    (reference forward.py:160-182 with save_argmax): the lowest index among the
    maximal scores over valid doc tokens, -1 when doc j has no valid token.
    Cross product: docs = Nd; KD (kd=True, D [Nq*K, Ld, d]): query i scores docs
    [i*K, (i+1)*K). float64 scores."""
    Q = np.asarray(Q, dtype=np.float64)
    D = np.asarray(D, dtype=np.float64)
    if normalize:
        Q, D = _normalize(Q), _normalize(D)
    Nq, Lq, _ = Q.shape
    Nd, Ld, _ = D.shape
    docs = Nd // Nq if kd else Nd
    dm = np.ones((Nd, Ld), bool) if d_mask is None else np.broadcast_to(np.asarray(d_mask, bool), (Nd, Ld))
    out = np.full((Nq * docs, Lq), -1, dtype=np.int64)
    for i in range(Nq):
        for jl in range(docs):
            j = i * docs + jl if kd else jl
            if not dm[j].any():
                continue
            S = Q[i] @ D[j].T  # [Lq, Ld]
            S = np.where(dm[j][None, :], S, NEG_INF)
            out[i * docs + jl] = S.argmax(axis=1)  # numpy argmax: first (lowest) index of the max
    return out


def maxsim_grads(G, Q, D, argmax, q_mask=None, *, normalize=False, kd=False):
    """Gradients of L = sum_ij G[i,j] * score[i,j] w.r.t. Q and D given the winners
    (reference backward/unified.py:27-88 plus the normalise Jacobian of
    autograd.py:211-225, with F.normalize's eps 1e-12):
      dL/dQh[i,s] = qm[i,s] sum_j G[i,j] Dh[j, a(i,j,s)]
      dL/dDh[j,t] = sum_{i,s: a(i,j,s)=t} qm[i,s] G[i,j] Qh[i,s]
      dL/dX = (dL/dXh - <dL/dXh, Xh> Xh) / max(||X||, 1e-12).  float64."""
    G = np.asarray(G, dtype=np.float64)
    Q = np.asarray(Q, dtype=np.float64)
    D = np.asarray(D, dtype=np.float64)
    Nq, Lq, d = Q.shape
    Nd, Ld, _ = D.shape
    docs = Nd // Nq if kd else Nd
    am = np.asarray(argmax).reshape(Nq, docs, Lq)
    qm = np.ones((Nq, Lq), bool) if q_mask is None else np.broadcast_to(np.asarray(q_mask, bool), (Nq, Lq))
    qn = np.maximum(np.sqrt((Q * Q).sum(-1, keepdims=True)), 1e-12)
    dn = np.maximum(np.sqrt((D * D).sum(-1, keepdims=True)), 1e-12)
    Qh, Dh = (Q / qn, D / dn) if normalize else (Q, D)
    gQh = np.zeros_like(Q)
    gDh = np.zeros_like(D)
    for i in range(Nq):
        for jl in range(docs):
            j = i * docs + jl if kd else jl
            for s in range(Lq):
                t = am[i, jl, s]
                if t < 0 or not qm[i, s]:
                    continue
                gQh[i, s] += G[i, jl] * Dh[j, t]
                gDh[j, t] += G[i, jl] * Qh[i, s]
    if not normalize:
        return gQh, gDh
    gQ = (gQh - (gQh * Qh).sum(-1, keepdims=True) * Qh) / qn
    gD = (gDh - (gDh * Dh).sum(-1, keepdims=True) * Dh) / dn
    return gQ, gD


def maxsim_kd(Q, D, q_mask=None, d_mask=None, *, normalize=False, dtype=np.float64):
    """KD layout Q [Nq, Lq, d] x D [Nq, K, Ld, d] -> [Nq, K]: query i against its own
    K docs (the per-query loop the reference tests use, tests/test_forward.py:318-320)."""
    Q = np.asarray(Q)
    D = np.asarray(D)
    Nq, K = D.shape[:2]
    out = np.zeros((Nq, K), dtype=dtype)
    for i in range(Nq):
        out[i] = maxsim(
            Q[i : i + 1], D[i],
            None if q_mask is None else np.asarray(q_mask)[i : i + 1],
            None if d_mask is None else np.asarray(d_mask)[i],
            normalize=normalize, dtype=dtype,
        )[0]
    return out


def _row_max_sum(S):
    """sum over query tokens of max over doc tokens, a non-finite max scoring 0.

    reference.py:83-85 applies the isfinite -> 0 rule in maxsim_reference; its
    packed / pair / padded loops (reference.py:236-306) sum the raw maxima, which
    differ only on non-finite inputs (a NaN or +inf similarity). Every entry point
    here scores like maxsim_reference, so that packed and padded inputs holding the
    same tokens give the same scores."""
    m = S.max(axis=1)
    return np.where(np.isfinite(m), m, 0.0).sum()


def maxsim_varlen(Qp, Dp, cu_q, cu_d, *, dtype=np.float64):
    """Packed MaxSim (reference.py:213-245): empty query or doc -> 0; a non-finite
    row max scores 0 (reference.py:83-85, see _row_max_sum)."""
    Qp = np.asarray(Qp, dtype=dtype)
    Dp = np.asarray(Dp, dtype=dtype)
    cu_q = np.asarray(cu_q, dtype=np.int64)
    cu_d = np.asarray(cu_d, dtype=np.int64)
    Nq, Nd = len(cu_q) - 1, len(cu_d) - 1
    out = np.zeros((Nq, Nd), dtype=dtype)
    for i in range(Nq):
        qi = Qp[cu_q[i] : cu_q[i + 1]]
        if qi.shape[0] == 0:
            continue
        for j in range(Nd):
            dj = Dp[cu_d[j] : cu_d[j + 1]]
            if dj.shape[0] == 0:
                continue
            out[i, j] = _row_max_sum(qi @ dj.T)
    return out


def maxsim_pairs(Qp, Dp, cu_q, cu_d, pair_q, pair_d, *, dtype=np.float64):
    """Pair-list MaxSim (reference.py:248-269)."""
    Qp = np.asarray(Qp, dtype=dtype)
    Dp = np.asarray(Dp, dtype=dtype)
    cu_q = np.asarray(cu_q, dtype=np.int64)
    cu_d = np.asarray(cu_d, dtype=np.int64)
    out = np.zeros(len(pair_q), dtype=dtype)
    for k, (i, j) in enumerate(zip(np.asarray(pair_q), np.asarray(pair_d))):
        qi = Qp[cu_q[i] : cu_q[i + 1]]
        dj = Dp[cu_d[j] : cu_d[j + 1]]
        if qi.shape[0] == 0 or dj.shape[0] == 0:
            continue
        out[k] = _row_max_sum(qi @ dj.T)
    return out


def maxsim_padded(queries, documents, query_lengths, doc_lengths, *, dtype=np.float64):
    """[B, Lq, d] x [B, C, Ld, d] with valid prefix lengths -> [B, C] (reference.py:272-306)."""
    Q = np.asarray(queries, dtype=dtype)
    D = np.asarray(documents, dtype=dtype)
    ql = np.asarray(query_lengths, dtype=np.int64)
    dl = np.asarray(doc_lengths, dtype=np.int64)
    B, C = D.shape[:2]
    out = np.zeros((B, C), dtype=dtype)
    for b in range(B):
        q = Q[b, : ql[b]]
        for c in range(C):
            dd = D[b, c, : dl[b, c]]
            if q.shape[0] == 0 or dd.shape[0] == 0:
                continue
            out[b, c] = _row_max_sum(q @ dd.T)
    return out


# --------------------------------------------------------------------------- #
# PLAID residuals                                                             #
# --------------------------------------------------------------------------- #


def unpack_residuals(residuals, nbits: int, d: int) -> np.ndarray:
    """Bucket code of feature f = (byte[f // cpb] >> ((f % cpb) * nbits)) & (2^nbits - 1),
    cpb = 8 // nbits: little-endian within each byte (reference.py:124-139)."""
    r = np.asarray(residuals, dtype=np.uint8).astype(np.int64)
    cpb = 8 // nbits
    mask = (1 << nbits) - 1
    f = np.arange(d)
    return (r[..., f // cpb] >> ((f % cpb) * nbits)) & mask


def pack_residuals(bucket_codes, nbits: int) -> np.ndarray:
    """Inverse of unpack_residuals: [..., d] codes -> [..., ceil(d*nbits/8)] uint8."""
    bc = np.asarray(bucket_codes, dtype=np.int64)
    d = bc.shape[-1]
    cpb = 8 // nbits
    pd = (d * nbits + 7) // 8
    out = np.zeros(bc.shape[:-1] + (pd,), dtype=np.int64)
    for f in range(d):
        out[..., f // cpb] |= bc[..., f] << ((f % cpb) * nbits)
    return out.astype(np.uint8)


def pack_residuals_colbert(bucket_codes, nbits: int) -> np.ndarray:
    """The on-disk residual encoding of ColBERTv2 / fast-plaid (third-party; not in
    the reference tree, whose loader reads these files at
    benchmarks/plaid/bench_fastplaid_e2e.py:75-140 and whose decoder notes the
    byte-reversed bit map at benchmarks/plaid/bench_decompress_maxsim.py:144-149):
    each code contributes its nbits bits least-significant first, and the bit
    stream is packed with numpy.packbits (first bit -> most significant bit)."""
    bc = np.asarray(bucket_codes, dtype=np.int64)
    bits = (bc[..., None] >> np.arange(nbits)) & 1  # [..., d, nbits], LSB first
    flat = bits.reshape(bc.shape[:-1] + (-1,)).astype(np.uint8)
    return np.packbits(flat, axis=-1)


def reverse_bits_bytes(b) -> np.ndarray:
    """Reverse the bit order of every byte (b7..b0 -> b0..b7)."""
    b = np.asarray(b, dtype=np.uint8)
    return np.unpackbits(b[..., None], axis=-1)[..., ::-1].reshape(b.shape + (8,)).dot(
        1 << np.arange(7, -1, -1)).astype(np.uint8)


def decode_residual_tokens(codes, residuals, centroids, bucket_weights, nbits: int, dtype=np.float64):
    """emb = centroids[code] + bucket_weights[clamp(bucket code)] (reference.py:158-163)."""
    cent = np.asarray(centroids, dtype=dtype)
    bw = np.asarray(bucket_weights, dtype=dtype)
    d = cent.shape[1]
    bc = np.clip(unpack_residuals(residuals, nbits, d), 0, bw.size - 1)
    return cent[np.asarray(codes, dtype=np.int64)] + bw[bc]


def maxsim_residual(Q, codes, residuals, doc_lengths, centroids, bucket_weights, nbits, *, normalize=True,
                    dtype=np.float64):
    """Padded decode + (normalise) + MaxSim (reference.py:142-179)."""
    Q = np.asarray(Q, dtype=dtype)
    if Q.ndim == 2:
        Q = Q[None]
    emb = decode_residual_tokens(codes, residuals, centroids, bucket_weights, nbits, dtype)
    L = emb.shape[1]
    dmask = np.arange(L)[None, :] < np.asarray(doc_lengths)[:, None]
    return maxsim(Q, emb, None, dmask, normalize=normalize, dtype=dtype)


def maxsim_residual_varlen(Q, codes_flat, residuals_flat, cu_seqlens_d, centroids, bucket_weights, nbits, *,
                           normalize=True, dtype=np.float64):
    """Ragged decode + MaxSim: the varlen twin of maxsim_residual (reference plaid.py:832-963)."""
    Q = np.asarray(Q, dtype=dtype)
    if Q.ndim == 2:
        Q = Q[None]
    emb = decode_residual_tokens(codes_flat, residuals_flat, centroids, bucket_weights, nbits, dtype)
    if normalize:
        emb = _normalize(emb)
        Q = _normalize(Q)
    Nq, Lq, d = Q.shape
    cu_q = np.arange(Nq + 1) * Lq
    return maxsim_varlen(Q.reshape(-1, d), emb, cu_q, cu_seqlens_d, dtype=dtype)


def plaid_approx_score(qcs, codes, doc_lengths, *, dtype=np.float64):
    """out[b] = sum_s max_{t < len_b} qcs[codes[b,t], s]; empty doc -> 0
    (reference.py:101-121; out-of-range codes clamp to 0 as in plaid.py:66-67)."""
    qcs = np.asarray(qcs, dtype=dtype)
    codes = np.asarray(codes, dtype=np.int64)
    n_cent = qcs.shape[0]
    codes = np.where((codes >= 0) & (codes < n_cent), codes, 0)
    B, L = codes.shape
    lens = np.asarray(doc_lengths, dtype=np.int64)
    g = qcs[codes.reshape(-1)].reshape(B, L, -1)
    mask = np.arange(L)[None, :] < lens[:, None]
    g = np.where(mask[:, :, None], g, NEG_INF)
    m = g.max(axis=1) if L > 0 else np.full((B, qcs.shape[1]), NEG_INF)
    m = np.where(np.isfinite(m), m, 0.0)
    return m.sum(axis=-1)


# --------------------------------------------------------------------------- #
# fp8 e4m3fn                                                                  #
# --------------------------------------------------------------------------- #

E4M3_MAX = 448.0


def _e4m3_table() -> np.ndarray:
    """All 127 non-negative finite e4m3fn values, ascending (bias 7, no inf,
    S.1111.111 is NaN; subnormals m * 2^-9)."""
    vals = []
    for e in range(16):
        for m in range(8):
            if e == 15 and m == 7:
                continue
            vals.append(m * 2.0**-9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7))
    return np.array(vals, dtype=np.float64)


_E4M3_POS = _e4m3_table()


def e4m3_round(x) -> np.ndarray:
    """Round to the nearest e4m3fn value, ties to even mantissa, saturating
    to +-448 (inputs are pre-clamped by the quantisers, fp8.py:44-46)."""
    x = np.asarray(x, dtype=np.float64)
    a = np.minimum(np.abs(x), E4M3_MAX)
    hi = np.searchsorted(_E4M3_POS, a, side="left")
    hi = np.clip(hi, 0, len(_E4M3_POS) - 1)
    lo = np.clip(hi - 1, 0, len(_E4M3_POS) - 1)
    vhi, vlo = _E4M3_POS[hi], _E4M3_POS[lo]
    dlo, dhi = a - vlo, vhi - a
    # ties: the table index parity is the mantissa parity (8 mantissas per exponent)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    r = np.where(a == vhi, vhi, np.where(pick_hi, vhi, vlo))
    return np.sign(x) * r


def quantize_fp8_per_tensor(X):
    """scale = max(amax, 1e-6) / 448; q = e4m3(clamp(x / scale, +-448)) (fp8.py:35-47).
    Returns (dequantised-grid values as float64, scale)."""
    X = np.asarray(X, dtype=np.float32)
    if X.size == 0:
        return X.astype(np.float64), np.float32(1.0)
    amax = np.float32(max(np.abs(X).max(), np.float32(1e-6)))
    scale = np.float32(amax / np.float32(E4M3_MAX))
    q = e4m3_round(np.clip((X / scale).astype(np.float32), -E4M3_MAX, E4M3_MAX))
    return q, scale


def quantize_fp8_per_token(X):
    """Per-row scale along the last axis (fp8.py:50-59)."""
    X = np.asarray(X, dtype=np.float32)
    amax = np.maximum(np.abs(X).max(axis=-1), np.float32(1e-6)).astype(np.float32)
    scale = (amax / np.float32(E4M3_MAX)).astype(np.float32)
    q = e4m3_round(np.clip((X / scale[..., None]).astype(np.float32), -E4M3_MAX, E4M3_MAX))
    return q, scale


# --------------------------------------------------------------------------- #
# top-k                                                                       #
# --------------------------------------------------------------------------- #


def topk_stable(scores, k: int, *, largest=True, index_base=0):
    """Top-k per row ordered by score (desc if largest) then lower index —
    the deterministic tie rule the north star fixes (torch.topk leaves it open)."""
    s = np.asarray(scores)
    k = min(k, s.shape[-1])
    key = -s if largest else s
    order = np.argsort(key, axis=-1, kind="stable")[..., :k]
    return np.take_along_axis(s, order, -1), order.astype(np.int64) + index_base


def retrieve_chunked(scores, k: int, chunk: int | None, *, largest=True):
    """Chunk-merge top-k over precomputed [Nq, Nd] scores, mirroring the loop of
    topk.py:54-86 / retrieve.py:284-305 (per-chunk top-k, concat with the
    running list, re-select min(k, width)) with the stable tie rule."""
    s = np.asarray(scores)
    Nd = s.shape[-1]
    k = min(k, Nd)
    if chunk is None or chunk >= Nd:
        return topk_stable(s, k, largest=largest)
    run_s = run_i = None
    for start in range(0, Nd, chunk):
        end = min(start + chunk, Nd)
        cs, ci = topk_stable(s[:, start:end], min(k, end - start), largest=largest, index_base=start)
        if run_s is None:
            run_s, run_i = cs, ci
        else:
            ms = np.concatenate([run_s, cs], -1)
            mi = np.concatenate([run_i, ci], -1)
            key = np.stack([mi, -ms if largest else ms])  # lexsort: last key primary
            order = np.lexsort(key, axis=-1)[..., : min(k, ms.shape[-1])]
            run_s = np.take_along_axis(ms, order, -1)
            run_i = np.take_along_axis(mi, order, -1)
    return run_s, run_i
