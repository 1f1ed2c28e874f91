"""``maxsim`` / ``maxsim_pairs``: the PyLate / colpali-engine "lik" entry points.

Signatures and dispatch follow the reference's ``autograd.py:356-501``:
``D.dim() == 4`` selects the KD layout (``[Nq, K, Ld, d]`` -> ``[Nq, K]``),
2-D inputs squeeze the matching output dim, masks are ``True`` = keep.
All scoring runs in the gfx950 HIP kernels of liblik_hip.so.

Gradients: when Q or D requires grad (and grad mode is on), the training
forward saves each winner's doc-token index and the backward runs the
deterministic HIP gradient kernels (``lik_maxsim_backward``). The
reference's ``backward="unified" | "lowmem"`` strategies both map to that
one implementation (atomic-free, bitwise reproducible); the argument is
validated for compatibility.
"""

from __future__ import annotations

import os
import warnings

import torch

from ._core import dense_maxsim, dense_maxsim_train, maxsim_backward, unify_dtype

_VALID_METHODS = ("auto", "unified", "lowmem")

# One-shot unnormalised-input check (reference autograd.py:136-166).
_NORM_CHECKED = False


def _validate_devices(Q, D, q_mask, d_mask) -> None:
    if Q.device != D.device:
        raise ValueError(
            f"Q and D must be on the same device; got Q.device={Q.device} vs D.device={D.device}."
        )
    if q_mask is not None and q_mask.device != Q.device:
        raise ValueError(f"q_mask must be on the same device as Q; got {q_mask.device} vs {Q.device}.")
    if d_mask is not None and d_mask.device != D.device:
        raise ValueError(f"d_mask must be on the same device as D; got {d_mask.device} vs {D.device}.")


def _maybe_warn_unnormalized(Q: torch.Tensor) -> None:
    """Warn once when ``normalize=False`` meets raw (non unit-norm) query tokens."""
    global _NORM_CHECKED
    if _NORM_CHECKED or os.environ.get("LIK_SUPPRESS_NORM_WARN", "0") == "1":
        return
    _NORM_CHECKED = True
    with torch.no_grad():
        sample = Q.detach().reshape(-1, Q.shape[-1])[:64]
        if sample.numel() == 0:
            return
        med = sample.float().norm(dim=-1).median().item()
    if not (0.9 <= med <= 1.1):
        warnings.warn(
            f"late-interaction-kernels: `maxsim(..., normalize=False)` but Q's median L2 norm "
            f"is {med:.3f} (ColBERT-style models expect ~1.0). Pass `normalize=True` to fuse "
            "the L2-norm into the kernel, or pre-normalize with `F.normalize(Q, dim=-1)`. "
            "Silence with `LIK_SUPPRESS_NORM_WARN=1`.",
            UserWarning,
            stacklevel=3,
        )


def _needs_grad(*ts: torch.Tensor) -> bool:
    return torch.is_grad_enabled() and any(t.requires_grad for t in ts)


class _MaxSimFn(torch.autograd.Function):
    """Fused MaxSim with saved argmax (reference autograd.py:169-229)."""

    @staticmethod
    def forward(ctx, Q, D, q_mask, d_mask, norm, kd):
        scores, argmax, Qp, Dp, qm = dense_maxsim_train(Q, D, q_mask, d_mask, norm=norm, kd=kd)
        ctx.save_for_backward(Qp, Dp, argmax, qm)
        ctx.norm = norm
        ctx.kd = kd
        ctx.shapes = (Q.shape, D.shape)
        ctx.dtypes = (Q.dtype, D.dtype)
        ctx.mark_non_differentiable(argmax)
        return scores

    @staticmethod
    def backward(ctx, grad_scores):
        Qp, Dp, argmax, qm = ctx.saved_tensors
        gq, gd = maxsim_backward(grad_scores, Qp, Dp, argmax, qm, norm=ctx.norm, kd=ctx.kd)
        (qshape, dshape), (qdt, ddt) = ctx.shapes, ctx.dtypes
        gq = gq[..., : qshape[-1]].to(qdt) if ctx.needs_input_grad[0] else None
        gd = gd[..., : dshape[-1]].to(ddt) if ctx.needs_input_grad[1] else None
        return gq, gd, None, None, None, None


def _score(Q, D, q_mask, d_mask, *, normalize: bool | int, kd: bool = False) -> torch.Tensor:
    """``normalize``: bool (both sides) or a bitmask (1: query tokens, 2: doc tokens)."""
    norm = (3 if normalize else 0) if isinstance(normalize, bool) else int(normalize)
    if _needs_grad(Q, D):
        if Q.dtype == torch.float64 or D.dtype == torch.float64:
            raise TypeError("maxsim gradients support fp16 / bf16 / fp32 inputs")
        return _MaxSimFn.apply(Q, D, q_mask, d_mask, norm, kd)
    return dense_maxsim(Q, D, q_mask, d_mask, norm=norm, kd=kd)


def _resolve_method(backward: str | None) -> str:
    if backward is None:
        return "auto"
    if backward not in _VALID_METHODS:
        raise ValueError(f"backward= must be one of {_VALID_METHODS} or None, got {backward!r}")
    return backward


def _maxsim_kd(Q, D, q_mask, d_mask, *, normalize: bool) -> torch.Tensor:
    """KD layout ``[Nq, Lq, d] x [Nq, K, Ld, d] -> [Nq, K]`` (reference autograd.py:232-287)."""
    if Q.dim() != 3:
        raise ValueError(f"KD layout (D.dim()==4) needs Q to be [Nq, Lq, d]; got Q.shape={tuple(Q.shape)}")
    Nq, Lq, d_q = Q.shape
    Nq_d, K, Ld, d_d = D.shape
    if Nq != Nq_d:
        raise ValueError(
            f"KD layout needs D.shape[0] == Q.shape[0]; got Q.shape[0]={Nq} vs D.shape[0]={Nq_d}."
        )
    if d_q != d_d:
        raise ValueError(f"Q and D must share the embedding dim; got {d_q} vs {d_d}.")
    if q_mask is not None and tuple(q_mask.shape) != (Nq, Lq):
        raise ValueError(f"q_mask must be [Nq={Nq}, Lq={Lq}] for KD layout; got {tuple(q_mask.shape)}.")
    if d_mask is not None and tuple(d_mask.shape) != (Nq, K, Ld):
        raise ValueError(
            f"d_mask must be [Nq={Nq}, K={K}, Ld={Ld}] for KD layout; got {tuple(d_mask.shape)}."
        )
    _validate_devices(Q, D, q_mask, d_mask)
    Q, D = unify_dtype(Q, D)
    D_flat = D.reshape(Nq * K, Ld, d_d)
    dm = d_mask.reshape(Nq * K, Ld) if d_mask is not None else None
    return _score(Q, D_flat, q_mask, dm, normalize=normalize, kd=True)


def maxsim(
    Q: torch.Tensor,
    D: torch.Tensor,
    q_mask: torch.Tensor | None = None,
    d_mask: torch.Tensor | None = None,
    *,
    normalize: bool = False,
    backward: str | None = None,
) -> torch.Tensor:
    """Fused MaxSim. Drop-in for PyLate's ``colbert_scores``.

    Args:
        Q: ``[Nq, Lq, d]`` or ``[Lq, d]``.
        D: ``[Ld, d]`` (single doc), ``[Nd, Ld, d]`` (in-batch cross product
            -> ``[Nq, Nd]``) or ``[Nq, K, Ld, d]`` (KD layout -> ``[Nq, K]``).
        q_mask, d_mask: bool masks, ``True`` = valid token. A dropped doc
            token never wins the max; a dropped query token adds nothing.
        normalize: L2-normalise Q and D per token inside the kernel.
        backward: ``"auto" | "unified" | "lowmem"`` or ``None`` (validated,
            see the module note).

    Returns:
        fp32 scores, shape as above. fp16/bf16 inputs are multiplied on the
        bf16/fp16 MFMA units with fp32 accumulation; fp32 inputs use a
        three-term bf16 split (~fp32 accuracy). Any Lq is supported: long
        queries are split into query-token chunks whose scores add up.
    """
    _resolve_method(backward)
    if D.dim() == 4:
        return _maxsim_kd(Q, D, q_mask, d_mask, normalize=normalize)

    q_was_2d = Q.dim() == 2
    d_was_2d = D.dim() == 2
    if q_was_2d:
        Q = Q.unsqueeze(0)
    if d_was_2d:
        D = D.unsqueeze(0)
    if q_mask is not None and q_mask.dim() == 1:
        q_mask = q_mask.unsqueeze(0)
    if d_mask is not None and d_mask.dim() == 1:
        d_mask = d_mask.unsqueeze(0)
    if Q.dim() != 3 or D.dim() != 3:
        raise ValueError(f"maxsim expects Q [Nq, Lq, d] and D [Nd, Ld, d]; got {tuple(Q.shape)}, {tuple(D.shape)}")
    if Q.shape[-1] != D.shape[-1]:
        raise ValueError(
            f"Q and D must share the embedding dim; got Q.shape[-1]={Q.shape[-1]} "
            f"vs D.shape[-1]={D.shape[-1]}."
        )
    _validate_devices(Q, D, q_mask, d_mask)
    if not normalize:
        _maybe_warn_unnormalized(Q)
    Q, D = unify_dtype(Q, D)
    scores = _score(Q, D, q_mask, d_mask, normalize=normalize)
    if q_was_2d and d_was_2d:
        return scores.reshape(())
    if q_was_2d:
        return scores.squeeze(0)
    if d_was_2d:
        return scores.squeeze(-1)
    return scores


def maxsim_pairs(
    Q: torch.Tensor,
    D: torch.Tensor,
    q_mask: torch.Tensor | None = None,
    d_mask: torch.Tensor | None = None,
    *,
    normalize: bool = False,
    backward: str | None = None,
) -> torch.Tensor:
    """Paired MaxSim ``score[i] = MaxSim(Q[i], D[i])`` -> ``[B]`` (PyLate's
    ``colbert_scores_pairwise``); the ``K = 1`` case of the KD layout."""
    if Q.dim() != 3 or D.dim() != 3:
        raise ValueError(
            f"maxsim_pairs needs both Q and D to be [B, L, d]; got Q.shape={tuple(Q.shape)}, "
            f"D.shape={tuple(D.shape)}."
        )
    if Q.shape[0] != D.shape[0]:
        raise ValueError(f"maxsim_pairs needs Q.shape[0] == D.shape[0]; got {Q.shape[0]} vs {D.shape[0]}.")
    D_kd = D.unsqueeze(1)
    d_mask_kd = d_mask.unsqueeze(1) if d_mask is not None else None
    out = maxsim(Q, D_kd, q_mask=q_mask, d_mask=d_mask_kd, normalize=normalize, backward=backward)
    return out.squeeze(-1)


__all__ = ["maxsim", "maxsim_pairs"]
