"""High-level entry points: :class:`MaxSimScorer` and :func:`retrieve` (reference retrieve.py).

Both default to ``normalize=True`` (ColBERT / ColPali convention) and run
the gfx950 kernels; inputs must be ROCm GPU tensors.
"""

from __future__ import annotations

from typing import Literal

import torch

from .autograd import maxsim
from .topk import maxsim_topk

BackwardMethod = Literal["auto", "unified", "lowmem"]
_VALID_METHODS: tuple[str, ...] = ("auto", "unified", "lowmem")


def _score(Q, D, q_mask, d_mask, *, normalize: bool, backward: str, inference: bool) -> torch.Tensor:
    if Q.device != D.device:
        raise ValueError(
            f"Q and D must be on the same device; got Q.device={Q.device} vs D.device={D.device}."
        )
    if inference:
        with torch.no_grad():
            return maxsim(Q, D, q_mask=q_mask, d_mask=d_mask, normalize=normalize, backward=backward)
    return maxsim(Q, D, q_mask=q_mask, d_mask=d_mask, normalize=normalize, backward=backward)


class MaxSimScorer(torch.nn.Module):
    """Stateless ``nn.Module`` for late-interaction (MaxSim) scoring.

    Args:
        normalize: L2-normalise Q and D per token inside the kernel.
        backward: gradient strategy name; ``"unified"`` and ``"lowmem"`` both map to
            the deterministic argmax-scatter backward (validated for compatibility).
        mask_pad_token: pad-token id for :meth:`forward_with_ids`.
    """

    def __init__(
        self,
        *,
        normalize: bool = True,
        backward: BackwardMethod = "auto",
        mask_pad_token: int | None = None,
    ) -> None:
        super().__init__()
        if backward not in _VALID_METHODS:
            raise ValueError(f"backward= must be one of {_VALID_METHODS}, got {backward!r}")
        self.normalize = normalize
        self.backward = backward
        self.mask_pad_token = mask_pad_token

    def extra_repr(self) -> str:
        return f"normalize={self.normalize}, backward={self.backward!r}, mask_pad_token={self.mask_pad_token!r}"

    def forward(self, Q, D, q_mask=None, d_mask=None) -> torch.Tensor:
        """MaxSim scores ``[Nq, Nd]``."""
        return _score(Q, D, q_mask, d_mask, normalize=self.normalize, backward=self.backward, inference=False)

    def score(self, Q, D, q_mask=None, d_mask=None) -> torch.Tensor:
        """Inference-only MaxSim (never participates in autograd)."""
        return _score(Q, D, q_mask, d_mask, normalize=self.normalize, backward=self.backward, inference=True)

    def retrieve(self, Q, D, top_k: int, q_mask=None, d_mask=None, *, chunk: int | None = None):
        """``(top_k_scores, top_k_indices)`` per query; see :func:`retrieve`."""
        return retrieve(Q, D, top_k=top_k, q_mask=q_mask, d_mask=d_mask, normalize=self.normalize, chunk=chunk)

    def forward_with_ids(self, Q, D, q_ids, d_ids) -> torch.Tensor:
        """Like :meth:`forward`, with masks ``q_ids != mask_pad_token`` / ``d_ids != mask_pad_token``."""
        if self.mask_pad_token is None:
            raise ValueError("`forward_with_ids` requires `mask_pad_token` set on the scorer.")
        return self.forward(Q, D, q_mask=q_ids != self.mask_pad_token, d_mask=d_ids != self.mask_pad_token)


def retrieve(
    Q: torch.Tensor,
    D: torch.Tensor,
    top_k: int,
    q_mask: torch.Tensor | None = None,
    d_mask: torch.Tensor | None = None,
    *,
    normalize: bool = True,
    chunk: int | None = None,
    largest: bool = True,
    sorted: bool = True,  # noqa: A002 - reference kwarg name
) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-``top_k`` late-interaction retrieval: ``(scores [Nq, k], indices [Nq, k])``.

    ``top_k`` is clamped to ``Nd``; ``chunk`` bounds the score buffer at
    ``Nq * chunk`` floats. Ties are broken by the lower document index, so the
    result does not depend on ``chunk``. Inference only.
    """
    if top_k <= 0:
        raise ValueError(f"top_k must be positive, got {top_k}")
    if Q.device != D.device:
        raise ValueError(
            f"Q and D must be on the same device; got Q.device={Q.device} vs D.device={D.device}."
        )
    return maxsim_topk(
        Q, D, k=top_k, q_mask=q_mask, d_mask=d_mask, normalize=normalize, chunk_size=chunk,
        largest=largest, sorted=sorted,
    )


__all__ = ["MaxSimScorer", "retrieve"]
