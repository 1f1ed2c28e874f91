"""FP8 (OCP e4m3fn) MaxSim inference (reference fp8.py).

``quantize_fp8_per_tensor`` / ``quantize_fp8_per_token`` follow
``fp8.py:35-59``: ``scale = amax / 448`` (amax clamped to >= 1e-6),
``x_fp8 = clamp(x / scale, +-448)`` cast with round-to-nearest-even.

``maxsim_inference_fp8`` runs the gfx950 fp8 MFMA kernel
(``v_mfma_scale_f32_32x32x64_f8f6f4``, fp32 accumulation). Per-tensor scales
are folded into one multiply of the final score (both scales are positive,
so ``max(s*x) = s*max(x)`` and the sum is linear); per-token scales scale the
rows before the max (doc side) or the per-token maxima (query side).
"""

from __future__ import annotations

import torch

from ._core import dense_maxsim
from .autograd import _validate_devices

_FP8_E4M3_MAX = 448.0
_E4M3 = getattr(torch, "float8_e4m3fn", None)
_E5M2 = getattr(torch, "float8_e5m2", None)


def quantize_fp8_per_tensor(X: torch.Tensor, dtype: torch.dtype | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize with one fp32 scale; dequantize as ``X_fp8.float() * scale``."""
    dtype = dtype or _E4M3
    if X.numel() == 0:
        return X.to(dtype), torch.ones((), device=X.device, dtype=torch.float32)
    amax = X.abs().amax().clamp_min(1e-6).to(torch.float32)
    scale = amax / _FP8_E4M3_MAX
    X_fp8 = (X.to(torch.float32) / scale).clamp(-_FP8_E4M3_MAX, _FP8_E4M3_MAX).to(dtype)
    return X_fp8.contiguous(), scale


def quantize_fp8_per_token(X: torch.Tensor, dtype: torch.dtype | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize each row (last axis) with its own scale; scale has shape ``X.shape[:-1]``."""
    dtype = dtype or _E4M3
    amax = X.abs().amax(dim=-1).clamp_min(1e-6).to(torch.float32)
    scale = amax / _FP8_E4M3_MAX
    X_fp8 = (X.to(torch.float32) / scale.unsqueeze(-1)).clamp(-_FP8_E4M3_MAX, _FP8_E4M3_MAX).to(dtype)
    return X_fp8.contiguous(), scale


def dequantize_fp8_per_tensor(X_fp8: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    return X_fp8.to(torch.float32) * scale


def dequantize_fp8_per_token(X_fp8: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    return X_fp8.to(torch.float32) * scale.unsqueeze(-1)


def maxsim_inference_fp8(
    Q: torch.Tensor,
    D: torch.Tensor,
    *,
    scale_Q: torch.Tensor,
    scale_D: torch.Tensor,
    q_mask: torch.Tensor | None = None,
    d_mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """MaxSim on fp8 inputs with per-tensor (0-d) or per-token (``[N, L]``) fp32 scales.

    Returns ``[Nq, Nd]`` fp32, squeezed for 2-D inputs. ``float8_e4m3fn`` runs
    on the fp8 MFMA path; ``float8_e5m2`` inputs are dequantised to bf16 and
    scored by the bf16 kernel. Per-tensor scales are read by the kernel from
    device memory (no host sync, graph-capturable; the reference reads them
    on the host).
    """
    q_was_2d = Q.dim() == 2
    d_was_2d = D.dim() == 2
    if q_was_2d:
        Q = Q.unsqueeze(0)
        if scale_Q.dim() > 0:
            scale_Q = scale_Q.unsqueeze(0)
    if d_was_2d:
        D = D.unsqueeze(0)
        if scale_D.dim() > 0:
            scale_D = scale_D.unsqueeze(0)
    if q_mask is not None and q_mask.dim() == 1:
        q_mask = q_mask.unsqueeze(0)
    if d_mask is not None and d_mask.dim() == 1:
        d_mask = d_mask.unsqueeze(0)
    if Q.shape[-1] != D.shape[-1]:
        raise ValueError(f"Q and D must share the embedding dim; got {Q.shape[-1]} vs {D.shape[-1]}.")
    _validate_devices(Q, D, q_mask, d_mask)

    q_tok = scale_Q.dim() >= 2
    d_tok = scale_D.dim() >= 2

    if Q.dtype == _E4M3 and D.dtype == _E4M3:
        # Per-tensor scales stay on the device: the kernel reads them in its
        # epilogue (score * s_q * s_d), so the call needs no host sync and can
        # be captured in a graph.
        scores = dense_maxsim(
            Q, D, q_mask, d_mask,
            q_scale=(scale_Q if q_tok else scale_Q.reshape(())).to(device=Q.device, dtype=torch.float32),
            d_scale=(scale_D if d_tok else scale_D.reshape(())).to(device=D.device, dtype=torch.float32),
        )
    elif Q.dtype in (_E4M3, _E5M2) and D.dtype in (_E4M3, _E5M2):
        Qd = Q.to(torch.float32) * (scale_Q.unsqueeze(-1) if q_tok else scale_Q.reshape(()))
        Dd = D.to(torch.float32) * (scale_D.unsqueeze(-1) if d_tok else scale_D.reshape(()))
        scores = dense_maxsim(Qd.to(torch.bfloat16), Dd.to(torch.bfloat16), q_mask, d_mask)
    else:
        raise TypeError(f"maxsim_inference_fp8 needs fp8 Q and D; got {Q.dtype} and {D.dtype}")

    if q_was_2d and d_was_2d:
        return scores.reshape(())
    if q_was_2d:
        return scores.squeeze(0)
    if d_was_2d:
        return scores.squeeze(-1)
    return scores


__all__ = [
    "maxsim_inference_fp8",
    "quantize_fp8_per_tensor",
    "quantize_fp8_per_token",
    "dequantize_fp8_per_tensor",
    "dequantize_fp8_per_token",
]
