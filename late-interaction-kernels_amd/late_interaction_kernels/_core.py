"""Shared launch path for the dense-embedding MaxSim entry points.

Every public scoring function (``maxsim``, ``maxsim_pairs``, ``maxsim_varlen``,
``maxsim_padded``, ``score_pairs_packed``, ``maxsim_inference_fp8``,
``retrieve``) normalises its inputs here and calls ``lik_maxsim`` /
``lik_maxsim_pairs`` from liblik_hip.so.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

_FP8 = getattr(torch, "float8_e4m3fn", None)


def unify_dtype(Q: torch.Tensor, D: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Pick one compute dtype for Q and D.

    bf16 if either side is bf16 (the reference's rule, ``_utils.py:137-148``),
    fp16 if both are fp16, otherwise fp32. fp32 is computed as a three-term
    bf16 split on the MFMA units (about 16 mantissa bits per product), where
    the reference truncates fp32 to fp16.
    """
    if Q.dtype == _FP8 or D.dtype == _FP8:
        raise TypeError("fp8 inputs go through late_interaction_kernels.fp8.maxsim_inference_fp8")
    if not (Q.is_floating_point() and D.is_floating_point()):
        raise TypeError(f"Q and D must be floating point; got {Q.dtype} and {D.dtype}")
    if torch.bfloat16 in (Q.dtype, D.dtype):
        t = torch.bfloat16
    elif Q.dtype == torch.float16 and D.dtype == torch.float16:
        t = torch.float16
    else:
        t = torch.float32
    return Q.to(t), D.to(t)


def _mask_i8(m: torch.Tensor | None, shape: tuple[int, int]) -> torch.Tensor | None:
    """Keep flags as int8 for the kernels, which read ``mask[i * sn + t * sl] != 0``
    with the tensor's own strides: a bool / 8-bit mask is reinterpreted in place
    (no copy, broadcast strides kept); other dtypes become ``m != 0``."""
    if m is None:
        return None
    if tuple(m.shape) != tuple(shape):
        m = m.expand(shape)
    if m.dtype == torch.int8:
        return m
    if m.dtype in (torch.bool, torch.uint8):
        return m.view(torch.int8)
    return (m != 0).view(torch.int8)


def _i32(t: torch.Tensor | None) -> torch.Tensor | None:
    return None if t is None else t.to(torch.int32).contiguous()


def dense_maxsim(
    Q: torch.Tensor,
    D: torch.Tensor,
    q_mask: torch.Tensor | None = None,
    d_mask: torch.Tensor | None = None,
    *,
    normalize: bool = False,
    norm: int | None = None,
    kd: bool = False,
    q_lengths: torch.Tensor | None = None,
    d_lengths: torch.Tensor | None = None,
    q_scale: torch.Tensor | None = None,
    d_scale: torch.Tensor | None = None,
    out_scale: float = 1.0,
) -> torch.Tensor:
    """``Q[Nq, Lq, d]`` x ``D[Nd, Ld, d]`` -> ``[Nq, Nd]`` fp32 (KD: ``D[Nq*K, Ld, d]`` -> ``[Nq, K]``).

    Masks are ``[N, L]`` keep-flags; lengths are valid prefix lengths per
    sequence; scales are fp8 per-token dequant scales ``[N, L]``.
    """
    _lib.require_gpu(Q, D, q_mask, d_mask, q_lengths, d_lengths, q_scale, d_scale)
    Nq, Lq, _ = Q.shape
    Nd, Ld, _ = D.shape
    Nd_eff = (Nd // Nq if Nq else 0) if kd else Nd
    out = torch.empty(Nq, Nd_eff, device=Q.device, dtype=torch.float32)
    if Nq == 0 or Nd_eff == 0:
        return out
    if Lq == 0 or Ld == 0:
        return out.zero_()
    Q = _lib.prepare_tokens(Q)
    D = _lib.prepare_tokens(D)
    qm = _mask_i8(q_mask, (Nq, Lq))
    dm = _mask_i8(d_mask, (Nd, Ld))
    ql = _i32(q_lengths)
    dl = _i32(d_lengths)
    # a 0-d scale is one per-tensor scale (strides 0: the kernel folds it
    # into the score scale); [N, L] scales are per token
    qsc = None if q_scale is None else (q_scale.to(torch.float32).reshape(1, 1) if q_scale.dim() == 0
                                        else q_scale.to(torch.float32).expand(Nq, Lq).contiguous())
    dsc = None if d_scale is None else (d_scale.to(torch.float32).reshape(1, 1) if d_scale.dim() == 0
                                        else d_scale.to(torch.float32).expand(Nd, Ld).contiguous())
    qs = _lib.seqs(
        Q, n=Nq, length=Lq, stride_n=Q.stride(0), stride_l=Q.stride(1), lengths=ql, mask=qm,
        mask_strides=(qm.stride(0), qm.stride(1)) if qm is not None else (0, 0),
        token_scale=qsc, scale_strides=(qsc.stride(0), qsc.stride(1)) if qsc is not None and qsc.numel() > 1 else (0, 0),
    )
    ds = _lib.seqs(
        D, n=Nd, length=Ld, stride_n=D.stride(0), stride_l=D.stride(1), lengths=dl, mask=dm,
        mask_strides=(dm.stride(0), dm.stride(1)) if dm is not None else (0, 0),
        token_scale=dsc, scale_strides=(dsc.stride(0), dsc.stride(1)) if dsc is not None and dsc.numel() > 1 else (0, 0),
    )
    if norm is None:
        norm = 3 if normalize else 0
    flags = _lib.norm_flags(norm) | (_lib.LIK_KD_LAYOUT if kd else 0)
    _launch(qs, ds, flags, out_scale, out, Q.device)
    return out


def dense_maxsim_train(
    Q: torch.Tensor,
    D: torch.Tensor,
    q_mask: torch.Tensor | None,
    d_mask: torch.Tensor | None,
    *,
    norm: int,
    kd: bool,
):
    """Training forward: scores plus the saved state the backward needs.
    ``norm`` is a bitmask: 1 normalises query tokens, 2 doc tokens.

    Returns ``(scores, argmax, Qp, Dp, qm)``: ``argmax`` is ``[Nq * docs, Lq]``
    int32 (winning doc-token index, -1 for rows without a valid doc token);
    ``Qp`` / ``Dp`` are the kernel-ready (16-byte-row) copies of Q and D and
    ``qm`` the int8 query mask.
    """
    _lib.require_gpu(Q, D, q_mask, d_mask)
    Nq, Lq, _ = Q.shape
    Nd, Ld, _ = D.shape
    docs = (Nd // Nq if Nq else 0) if kd else Nd
    out = torch.empty(Nq, docs, device=Q.device, dtype=torch.float32)
    argmax = torch.full((Nq * docs, Lq), -1, device=Q.device, dtype=torch.int32)
    Qp = _lib.prepare_tokens(Q.detach())
    Dp = _lib.prepare_tokens(D.detach())
    qm = _mask_i8(q_mask, (Nq, Lq))
    if Nq == 0 or docs == 0 or Lq == 0 or Ld == 0:
        return out.zero_(), argmax, Qp, Dp, qm
    dm = _mask_i8(d_mask, (Nd, Ld))
    qs = _lib.seqs(Qp, n=Nq, length=Lq, stride_n=Qp.stride(0), stride_l=Qp.stride(1), mask=qm,
                   mask_strides=(qm.stride(0), qm.stride(1)) if qm is not None else (0, 0))
    ds = _lib.seqs(Dp, n=Nd, length=Ld, stride_n=Dp.stride(0), stride_l=Dp.stride(1), mask=dm,
                   mask_strides=(dm.stride(0), dm.stride(1)) if dm is not None else (0, 0))
    flags = _lib.norm_flags(norm) | (_lib.LIK_KD_LAYOUT if kd else 0)
    lib = _lib.load()
    nbytes = lib.lik_maxsim_workspace_size(ctypes.byref(qs), ctypes.byref(ds), flags)
    ws = _lib.workspace(nbytes, Q.device)
    with torch.cuda.device(Q.device):
        rc = lib.lik_maxsim_argmax(ctypes.byref(qs), ctypes.byref(ds), flags, out.data_ptr(), out.stride(0),
                                   out.stride(1), argmax.data_ptr(), _lib.ptr(ws), nbytes, _lib.stream_of(out))
    _lib.check(rc, "lik_maxsim_argmax")
    return out, argmax, Qp, Dp, qm


def maxsim_backward(
    grad: torch.Tensor,
    Qp: torch.Tensor,
    Dp: torch.Tensor,
    argmax: torch.Tensor,
    qm: torch.Tensor | None,
    *,
    norm: int,
    kd: bool,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(grad_Q [Nq, Lq, dp], grad_D [Nd, Ld, dp])`` in the input dtype for upstream ``grad`` [Nq, docs]."""
    Nq, Lq, dp = Qp.shape
    Nd, Ld, _ = Dp.shape
    if Nq == 0 or Nd == 0 or Lq == 0 or Ld == 0:
        return torch.zeros_like(Qp), torch.zeros_like(Dp)
    gq = torch.empty(Nq, Lq, dp, device=Qp.device, dtype=Qp.dtype)  # every element is written
    gd = torch.empty(Nd, Ld, dp, device=Dp.device, dtype=Dp.dtype)
    g = grad.to(torch.float32).contiguous()
    qs = _lib.seqs(Qp, n=Nq, length=Lq, stride_n=Qp.stride(0), stride_l=Qp.stride(1), mask=qm,
                   mask_strides=(qm.stride(0), qm.stride(1)) if qm is not None else (0, 0))
    ds = _lib.seqs(Dp, n=Nd, length=Ld, stride_n=Dp.stride(0), stride_l=Dp.stride(1))
    flags = _lib.norm_flags(norm) | (_lib.LIK_KD_LAYOUT if kd else 0)
    lib = _lib.load()
    nbytes = lib.lik_maxsim_backward_workspace_size(ctypes.byref(qs), ctypes.byref(ds), flags)
    ws = _lib.workspace(nbytes, Qp.device)
    with torch.cuda.device(Qp.device):
        rc = lib.lik_maxsim_backward(g.data_ptr(), g.stride(0), ctypes.byref(qs), ctypes.byref(ds), argmax.data_ptr(),
                                     flags, gq.data_ptr(), gd.data_ptr(), _lib.ptr(ws), nbytes,
                                     _lib.stream_of(gq))
    _lib.check(rc, "lik_maxsim_backward")
    return gq, gd


def packed_maxsim(
    Q_packed: torch.Tensor,
    D_packed: torch.Tensor,
    cu_q: torch.Tensor,
    cu_d: torch.Tensor,
    max_q: int,
    max_d: int,
    *,
    normalize: bool = False,
) -> torch.Tensor:
    """Packed (cu_seqlens) Q and D -> ``[Nq, Nd]`` fp32."""
    _lib.require_gpu(Q_packed, D_packed, cu_q, cu_d)
    Nq = cu_q.numel() - 1
    Nd = cu_d.numel() - 1
    out = torch.empty(max(Nq, 0), max(Nd, 0), device=Q_packed.device, dtype=torch.float32)
    if Nq <= 0 or Nd <= 0:
        return out
    if max_q <= 0 or Q_packed.shape[0] == 0 or D_packed.shape[0] == 0:
        return out.zero_()
    Qp = _lib.prepare_tokens(Q_packed)
    Dp = _lib.prepare_tokens(D_packed)
    cq = _i32(cu_q)
    cd = _i32(cu_d)
    # max_d is not a kernel bound (each doc's tile loop ends at its own length)
    qs = _lib.seqs(Qp, n=Nq, length=max_q, stride_l=Qp.stride(0), cu=cq)
    ds = _lib.seqs(Dp, n=Nd, length=max(int(max_d), 0), stride_l=Dp.stride(0), cu=cd)
    flags = _lib.LIK_NORMALIZE if normalize else 0
    _launch(qs, ds, flags, 1.0, out, Q_packed.device)
    return out


def packed_maxsim_train(Q_packed, D_packed, cu_q, cu_d, max_q: int, max_d: int):
    """Training forward on packed Q and D: ``(scores [Nq, Nd], argmax [Nq*Nd, max_q], Qp, Dp)``."""
    _lib.require_gpu(Q_packed, D_packed, cu_q, cu_d)
    Nq = cu_q.numel() - 1
    Nd = cu_d.numel() - 1
    out = torch.zeros(max(Nq, 0), max(Nd, 0), device=Q_packed.device, dtype=torch.float32)
    argmax = torch.full((max(Nq, 0) * max(Nd, 0), max(max_q, 0)), -1, device=Q_packed.device, dtype=torch.int32)
    Qp = _lib.prepare_tokens(Q_packed.detach())
    Dp = _lib.prepare_tokens(D_packed.detach())
    if Nq <= 0 or Nd <= 0 or max_q <= 0 or Q_packed.shape[0] == 0 or D_packed.shape[0] == 0:
        return out, argmax, Qp, Dp
    qs = _lib.seqs(Qp, n=Nq, length=max_q, stride_l=Qp.stride(0), cu=cu_q)
    ds = _lib.seqs(Dp, n=Nd, length=max(int(max_d), 0), stride_l=Dp.stride(0), cu=cu_d)
    lib = _lib.load()
    nbytes = lib.lik_maxsim_workspace_size(ctypes.byref(qs), ctypes.byref(ds), 0)
    ws = _lib.workspace(nbytes, Q_packed.device)
    with torch.cuda.device(Q_packed.device):
        rc = lib.lik_maxsim_argmax(ctypes.byref(qs), ctypes.byref(ds), 0, out.data_ptr(), out.stride(0),
                                   out.stride(1), argmax.data_ptr(), _lib.ptr(ws), nbytes, _lib.stream_of(out))
    _lib.check(rc, "lik_maxsim_argmax")
    return out, argmax, Qp, Dp


def packed_backward(grad, Qp, Dp, cu_q, cu_d, argmax, max_q: int, max_d: int, *, need_d: bool = True):
    """Gradients of packed MaxSim: ``(grad_Q [rows_q, dp], grad_D [rows_d, dp] or None)`` in the input dtype.
    Rows outside ``cu[0] .. cu[-1]`` are zero."""
    Nq = cu_q.numel() - 1
    Nd = cu_d.numel() - 1
    gq = torch.zeros_like(Qp)
    gd = torch.zeros_like(Dp) if need_d else None
    if Nq <= 0 or Nd <= 0 or max_q <= 0 or Qp.shape[0] == 0 or Dp.shape[0] == 0:
        return gq, gd
    g = grad.to(torch.float32).contiguous()
    qs = _lib.seqs(Qp, n=Nq, length=max_q, stride_l=Qp.stride(0), cu=cu_q)
    ds = _lib.seqs(Dp, n=Nd, length=max(int(max_d), 0), stride_l=Dp.stride(0), cu=cu_d)
    lib = _lib.load()
    nbytes = lib.lik_maxsim_backward_workspace_size(ctypes.byref(qs), ctypes.byref(ds), 0)
    ws = _lib.workspace(nbytes, Qp.device)
    with torch.cuda.device(Qp.device):
        rc = lib.lik_maxsim_backward(g.data_ptr(), g.stride(0), ctypes.byref(qs), ctypes.byref(ds), argmax.data_ptr(),
                                     0, gq.data_ptr(), _lib.ptr(gd), _lib.ptr(ws), nbytes, _lib.stream_of(gq))
    _lib.check(rc, "lik_maxsim_backward")
    return gq, gd


def _launch(qs, ds, flags: int, out_scale: float, out: torch.Tensor, device: torch.device) -> None:
    lib = _lib.load()
    opts = _lib.call_opts()
    nbytes = lib.lik_maxsim_workspace_size_ex(ctypes.byref(qs), ctypes.byref(ds), flags, opts)
    ws = _lib.workspace(nbytes, device)
    with torch.cuda.device(device):
        rc = lib.lik_maxsim_ex(
            ctypes.byref(qs), ctypes.byref(ds), flags, float(out_scale), out.data_ptr(), out.stride(0),
            out.stride(1), _lib.ptr(ws), nbytes, opts, _lib.stream_of(out),
        )
    _lib.check(rc, "lik_maxsim")


def pairs_maxsim(
    Q_packed: torch.Tensor,
    D_packed: torch.Tensor,
    cu_q: torch.Tensor,
    cu_d: torch.Tensor,
    pair_q: torch.Tensor,
    pair_d: torch.Tensor,
    max_q: int,
    max_d: int,
) -> torch.Tensor:
    """Pair-list MaxSim over packed Q and D -> ``[num_pairs]`` fp32."""
    _lib.require_gpu(Q_packed, D_packed, cu_q, cu_d, pair_q, pair_d)
    P = pair_q.numel()
    out = torch.empty(P, device=Q_packed.device, dtype=torch.float32)
    if P == 0:
        return out
    if max_q <= 0 or Q_packed.shape[0] == 0 or D_packed.shape[0] == 0:
        return out.zero_()
    Qp = _lib.prepare_tokens(Q_packed)
    Dp = _lib.prepare_tokens(D_packed)
    cq, cd, pq, pd = _i32(cu_q), _i32(cu_d), _i32(pair_q), _i32(pair_d)
    qs = _lib.seqs(Qp, n=cq.numel() - 1, length=max_q, stride_l=Qp.stride(0), cu=cq)
    ds = _lib.seqs(Dp, n=cd.numel() - 1, length=max(int(max_d), 0), stride_l=Dp.stride(0), cu=cd)
    lib = _lib.load()
    with torch.cuda.device(Q_packed.device):
        rc = lib.lik_maxsim_pairs(
            ctypes.byref(qs), ctypes.byref(ds), pq.data_ptr(), pd.data_ptr(), P, 0, out.data_ptr(),
            _lib.stream_of(out),
        )
    _lib.check(rc, "lik_maxsim_pairs")
    return out


def pairs_maxsim_train(Q_packed, D_packed, cu_q, cu_d, pair_q, pair_d, max_q: int, max_d: int):
    """Pair-list training forward: ``(scores [P], argmax [P, max_q], Qp, Dp)``."""
    _lib.require_gpu(Q_packed, D_packed, cu_q, cu_d, pair_q, pair_d)
    P = pair_q.numel()
    out = torch.zeros(P, device=Q_packed.device, dtype=torch.float32)
    argmax = torch.full((P, max(max_q, 0)), -1, device=Q_packed.device, dtype=torch.int32)
    Qp = _lib.prepare_tokens(Q_packed.detach())
    Dp = _lib.prepare_tokens(D_packed.detach())
    if P == 0 or max_q <= 0 or Q_packed.shape[0] == 0 or D_packed.shape[0] == 0:
        return out, argmax, Qp, Dp
    qs = _lib.seqs(Qp, n=cu_q.numel() - 1, length=max_q, stride_l=Qp.stride(0), cu=cu_q)
    ds = _lib.seqs(Dp, n=cu_d.numel() - 1, length=max(int(max_d), 0), stride_l=Dp.stride(0), cu=cu_d)
    lib = _lib.load()
    with torch.cuda.device(Q_packed.device):
        rc = lib.lik_maxsim_pairs_argmax(ctypes.byref(qs), ctypes.byref(ds), pair_q.data_ptr(), pair_d.data_ptr(), P,
                                         0, out.data_ptr(), argmax.data_ptr(), _lib.stream_of(out))
    _lib.check(rc, "lik_maxsim_pairs_argmax")
    return out, argmax, Qp, Dp


def pairs_backward(grad, Qp, Dp, cu_q, cu_d, pair_q, pair_d, argmax, max_q: int, max_d: int, *,
                   need_d: bool = True):
    """Gradients of pair-list MaxSim: ``(grad_Q [rows_q, dp], grad_D [rows_d, dp] or None)``."""
    P = pair_q.numel()
    gq = torch.zeros_like(Qp)
    gd = torch.zeros_like(Dp) if need_d else None
    if P == 0 or max_q <= 0 or Qp.shape[0] == 0 or Dp.shape[0] == 0:
        return gq, gd
    g = grad.to(torch.float32).contiguous()
    qs = _lib.seqs(Qp, n=cu_q.numel() - 1, length=max_q, stride_l=Qp.stride(0), cu=cu_q)
    ds = _lib.seqs(Dp, n=cu_d.numel() - 1, length=max(int(max_d), 0), stride_l=Dp.stride(0), cu=cu_d)
    lib = _lib.load()
    nbytes = lib.lik_maxsim_pairs_backward_workspace_size(ctypes.byref(qs), ctypes.byref(ds), P)
    ws = _lib.workspace(nbytes, Qp.device)
    with torch.cuda.device(Qp.device):
        rc = lib.lik_maxsim_pairs_backward(g.data_ptr(), ctypes.byref(qs), ctypes.byref(ds), pair_q.data_ptr(),
                                           pair_d.data_ptr(), P, argmax.data_ptr(), 0, gq.data_ptr(), _lib.ptr(gd),
                                           _lib.ptr(ws), nbytes, _lib.stream_of(gq))
    _lib.check(rc, "lik_maxsim_pairs_backward")
    return gq, gd


def seqlen_max(cu: torch.Tensor) -> int:
    """Longest sequence in ``cu_seqlens`` (one device->host sync)."""
    if cu.numel() <= 1:
        return 0
    return int((cu[1:] - cu[:-1]).max().item())


def assert_max_seqlen_covers(cu: torch.Tensor, max_seqlen: int, name: str) -> None:
    """On-device check that a caller-supplied bound covers every sequence
    (``_utils.py:32-50``): the bound sizes the query block, so a too-small
    value would drop tokens."""
    if cu.numel() <= 1:
        return
    torch._assert_async(
        (cu[1:] - cu[:-1]).max().le(max_seqlen),
        f"{name}={max_seqlen} is smaller than the longest sequence in cu_seqlens; "
        "it is a hard bound and would silently truncate tokens.",
    )


def from_hidden_forward(Q, H, W, b, d_mask, *, normalize: bool, want_argmax: bool):
    """Projection head fused into MaxSim (``lik_maxsim_from_hidden``): scores of
    ``Q [Nq, Lq, d_out]`` against ``normalize(H @ W^T + b)`` for ``H [Nd, Ld, d_model]``
    without forming the projected docs. Returns ``(scores, argmax or None)``, or
    ``None`` when the library reports the shape or dtype unsupported (the
    caller then projects first)."""
    _lib.require_gpu(Q, H, W, b, d_mask)
    if not (Q.dtype == H.dtype == W.dtype and Q.dtype in (torch.bfloat16, torch.float16)):
        return None
    Nq, Lq, d_out = Q.shape
    Nd, Ld, _ = H.shape
    # head_finish_kernel writes every score (and every argmax entry)
    out = torch.empty(Nq, Nd, device=Q.device, dtype=torch.float32)
    argmax = torch.empty((Nq * Nd, Lq), device=Q.device, dtype=torch.int32) if want_argmax else None
    Qc = Q.detach().contiguous()
    Hc = H.detach()
    if Hc.stride(-1) != 1 or Hc.data_ptr() % 16 or any(s % 8 for s in Hc.stride()[:-1]):
        Hc = Hc.contiguous()
    Wc = W.detach().contiguous()
    # a bias in the inputs' 16-bit dtype is read and widened by the kernel
    bias16 = b is not None and b.dtype == Q.dtype
    bias = None if b is None else (b.detach().contiguous() if bias16 else b.detach().to(torch.float32).contiguous())
    dm = _mask_i8(d_mask, (Nd, Ld))
    qs = _lib.seqs(Qc, n=Nq, length=Lq, stride_n=Qc.stride(0), stride_l=Qc.stride(1))
    hs = _lib.seqs(Hc, n=Nd, length=Ld, stride_n=Hc.stride(0), stride_l=Hc.stride(1), mask=dm,
                   mask_strides=(dm.stride(0), dm.stride(1)) if dm is not None else (0, 0))
    lib = _lib.load()
    nbytes = lib.lik_maxsim_from_hidden_workspace_size(ctypes.byref(qs), ctypes.byref(hs))
    ws = _lib.workspace(nbytes, Q.device)
    flags = (_lib.LIK_NORMALIZE_D if normalize else 0) | (_lib.LIK_BIAS_16 if bias16 else 0)
    with torch.cuda.device(Q.device):
        rc = lib.lik_maxsim_from_hidden(ctypes.byref(qs), ctypes.byref(hs), Wc.data_ptr(), Wc.stride(0),
                                        _lib.ptr(bias), flags, out.data_ptr(), out.stride(0), out.stride(1),
                                        _lib.ptr(argmax), _lib.ptr(ws), nbytes, _lib.stream_of(out))
    if rc == _lib.LIK_ERR_UNSUPPORTED:
        return None
    _lib.check(rc, "lik_maxsim_from_hidden")
    return out, argmax

