"""``maxsim_from_hidden``: MaxSim with the doc-side projection head in front
(reference fused_head.py:262-332).

Computes ``maxsim(Q, normalize(F.linear(H_d, W, b)))``; Q is taken as already
projected and normalised, as in the reference.

Inference (nothing requires grad): one HIP kernel (``lik_maxsim_from_hidden``)
projects each 32-token tile of H on the MFMA units, adds the bias, normalises
and rounds the rows in registers and scores them against the queries: the
projected docs never reach memory (reference fused_head.py:46-189). Shapes
the kernel does not take (fp32 inputs, d_out > 128, more than 256 query
tokens) project with one GEMM (``F.linear``) and score the materialised docs.

Training: the projection is one GEMM, then the argmax-saving MaxSim kernel
with the doc-only normalise. Only doc tokens that won some query token's max
have a gradient, so the projection's gradients are taken on those rows alone:
grad_W = g^T H_win, grad_b = sum g and grad_H = g W scattered into a zeroed
tensor (the reference's backward, fused_head.py:347-460, gathers H at the
winners the same way). Projecting first is the faster training route here:
with the fused forward, the backward has to gather and project the winning
rows again, and those extra small launches cost more than the fused forward
saves on the reference's training shapes.

The training route rounds the projection to the input dtype before it is
normalised (one bf16 GEMM); the inference kernel, like the reference's fused
kernel (fused_head.py:146-158), projects, adds the bias and normalises in fp32
and rounds once. Scores of the two routes differ by that rounding
(tests/test_gpu_fused_head.py compares them within 1e-2).
"""

from __future__ import annotations

import torch

from .autograd import _needs_grad, _score, _validate_devices
from ._core import dense_maxsim_train, from_hidden_forward, maxsim_backward, unify_dtype


class _FromHiddenFn(torch.autograd.Function):
    """Projection + MaxSim with the projection's gradients on winning rows only."""

    @staticmethod
    def forward(ctx, Q, H_d, W, b, d_mask, normalize):
        D = torch.nn.functional.linear(H_d.detach(), W.detach(), None if b is None else b.detach())
        Qc, Dc = unify_dtype(Q.detach(), D)
        norm = 2 if normalize else 0
        scores, argmax, Qp, Dp, qm = dense_maxsim_train(Qc, Dc, None, d_mask, norm=norm, kd=False)
        ctx.save_for_backward(Qp, Dp, argmax, H_d, W)
        ctx.norm = norm
        ctx.q_dtype = Q.dtype
        ctx.has_b = b is not None
        ctx.b_dtype = None if b is None else b.dtype
        return scores

    @staticmethod
    def backward(ctx, G):
        Qp, Dp, argmax, H_d, W = ctx.saved_tensors
        gq, gd = maxsim_backward(G, Qp, Dp, argmax, None, norm=ctx.norm, kd=False)
        Nq, Lq, d_out = Qp.shape[0], Qp.shape[1], W.shape[0]
        Nd, Ld, d_model = H_d.shape
        grad_q = gq[..., :d_out].to(ctx.q_dtype) if ctx.needs_input_grad[0] else None
        # doc rows that won a max (the only rows with a nonzero grad_D)
        am = argmax.view(Nq, Nd, Lq)
        rows = (torch.arange(Nd, device=am.device).view(1, Nd, 1) * Ld + am.long())[am >= 0]
        rows = torch.unique(rows)
        g_rows = gd.reshape(Nd * Ld, -1)[rows, :d_out].float()
        grad_h = grad_w = grad_b = None
        if ctx.needs_input_grad[1]:
            # dense (row-major) whatever H_d's strides: the rows are scattered through a view
            grad_h = torch.zeros(H_d.shape, dtype=H_d.dtype, device=H_d.device)
            grad_h.view(Nd * Ld, d_model)[rows] = (g_rows @ W.float()).to(H_d.dtype)
        if ctx.needs_input_grad[2]:
            grad_w = (g_rows.t() @ H_d.reshape(Nd * Ld, d_model)[rows].float()).to(W.dtype)
        if ctx.has_b and ctx.needs_input_grad[3]:
            grad_b = g_rows.sum(0).to(ctx.b_dtype)
        return grad_q, grad_h, grad_w, grad_b, None, None


def maxsim_from_hidden(
    Q: torch.Tensor,
    H_d: torch.Tensor,
    W: torch.Tensor,
    b: torch.Tensor | None = None,
    d_mask: torch.Tensor | None = None,
    normalize: bool = True,
) -> torch.Tensor:
    """``Q [Lq, d_out] | [Nq, Lq, d_out]``, ``H_d [Nd, Ld, d_model]``, ``W [d_out, d_model]``,
    ``b [d_out]`` -> fp32 scores ``[Nq, Nd]`` (``[Nd]`` for 2-D Q)."""
    q_was_2d = Q.dim() == 2
    if q_was_2d:
        Q = Q.unsqueeze(0)
    if d_mask is not None and d_mask.dim() == 1:
        d_mask = d_mask.unsqueeze(0)
    if Q.dim() != 3:
        raise ValueError(f"Q must be [Lq, d_out] or [Nq, Lq, d_out]; got {Q.shape}")
    if H_d.dim() != 3:
        raise ValueError(f"H_d must be [Nd, Ld, d_model]; got {H_d.shape}")
    if W.dim() != 2 or W.shape != (Q.shape[-1], H_d.shape[-1]):
        raise ValueError(f"W must be [d_out={Q.shape[-1]}, d_model={H_d.shape[-1]}]; got {W.shape}")
    if Q.device != H_d.device or W.device != Q.device:
        raise ValueError("Q, H_d, W must be on the same device.")
    if b is not None and (b.dim() != 1 or b.shape[0] != Q.shape[-1]):
        raise ValueError(f"b must be [d_out={Q.shape[-1]}]; got {tuple(b.shape) if b is not None else None}")
    _validate_devices(Q, H_d, None, d_mask)
    if _needs_grad(*(t for t in (Q, H_d, W, b) if t is not None)):
        if torch.float64 in (Q.dtype, H_d.dtype, W.dtype):
            raise TypeError("maxsim_from_hidden gradients support fp16 / bf16 / fp32 inputs")
        scores = _FromHiddenFn.apply(Q, H_d, W, b, d_mask, bool(normalize))
    else:
        fused = from_hidden_forward(Q, H_d, W, b, d_mask, normalize=bool(normalize), want_argmax=False)
        if fused is not None:
            scores = fused[0]
        else:
            D = torch.nn.functional.linear(H_d, W, b)
            Qc, Dc = unify_dtype(Q, D)
            scores = _score(Qc, Dc, None, d_mask, normalize=2 if normalize else 0)
    return scores.squeeze(0) if q_was_2d else scores


__all__ = ["maxsim_from_hidden"]
