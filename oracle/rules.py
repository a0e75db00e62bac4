"""Selection rules of the reference restated (src/attention_lab/selection.py:21-86). Test infrastructure only."""
from __future__ import annotations

import math

PREFIX, RECENT = 4, 64


def legal(query_position: int, valid_length: int) -> int:
    """selection.py:21-30: legal range [0, n), n = min(valid, qp + 1) >= 1."""
    if query_position < 0 or valid_length < 0:
        raise ValueError("negative position")
    n = min(valid_length, query_position + 1)
    if n <= 0:
        raise ValueError("no legal position")
    return n


def layout(n: int, prefix: int = PREFIX, recent: int = RECENT):
    """selection.py:69-77 -> (lo, hi): F = [0, lo) U [hi, n), candidates [lo, hi)."""
    if n <= 0:
        raise ValueError("legal length must be positive")
    lo = min(prefix, n)
    hi = max(lo, n - recent)
    return lo, hi


def budget(n0: int, rho: float, prefix: int = PREFIX, recent: int = RECENT) -> int:
    """selection.py:80-86: k0 = min(round(rho * n0), candidates at n0), Python round (ties to even)."""
    if math.isnan(rho) or not 0.0 <= rho <= 1.0:
        raise ValueError("rho must be in [0, 1]")
    lo, hi = layout(n0, prefix, recent)
    return min(round(rho * n0), hi - lo)


def step(n: int, k0: int):
    """(lo, hi, k, S) of a decode step with legal length n and request budget k0 (qwen_wrap.py:169-181)."""
    lo, hi = layout(n)
    k = min(k0, hi - lo)
    return lo, hi, k, lo + (n - hi) + k


def fixed_positions(n: int):
    lo, hi = layout(n)
    return list(range(lo)) + list(range(hi, n))
