"""Small helpers kept for API parity with the reference's ``_utils.py``."""

from __future__ import annotations


def next_pow2(x: int) -> int:
    """Smallest power of two >= x (``next_pow2(0) == 1``)."""
    if x <= 1:
        return 1
    return 1 << (x - 1).bit_length()


def bucket_seqlen(max_len: int, floor: int = 16) -> int:
    """Round a max sequence length up to a power of two (>= floor); 0 stays 0."""
    if max_len <= 0:
        return 0
    return max(floor, next_pow2(max_len))
