"""Read-set rules of one decode step: legal range, fixed set F, candidate domain and the budget k.

Same rules and public names as the reference's selection module (src/attention_lab/selection.py:17-86):

* positions [0, legal) are legal for the query, legal = min(valid_length, query_position + 1);
* F = the first FIXED_PREFIX legal positions plus the last FIXED_RECENT, which never overlap;
* the candidates are the one contiguous range [lo, hi) between them;
* k0 = min(round(rho * n0), candidates at n0) is fixed per request (Python's round: ties to even), and each step
  reads k = min(k0, candidates now) of them. Positions are never renumbered.

Pure Python; the HIP kernels receive lo, hi, legal and k as integers.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

FIXED_PREFIX = 4
FIXED_RECENT = 64


def legal_length(query_position: int, valid_length: int) -> int:
    """Size of the legal range [0, n) for a query at `query_position` over a cache holding `valid_length` keys."""
    qp, vl = int(query_position), int(valid_length)
    if qp < 0 or vl < 0:
        raise ValueError(f"negative query_position={qp} or valid_length={vl}")
    n = min(vl, qp + 1)
    if n < 1:
        raise ValueError(f"no legal key position for query_position={qp}, valid_length={vl}")
    return n


@dataclass(frozen=True)
class SelectionLayout:
    """Placement of F and the candidate domain inside [0, legal_length)."""

    legal_length: int
    fixed_prefix: int   # F's leading part is [0, fixed_prefix)
    recent_start: int   # F's trailing part is [recent_start, legal_length)

    @property
    def candidate_lo(self) -> int:
        return self.fixed_prefix

    @property
    def candidate_hi(self) -> int:
        return self.recent_start

    @property
    def candidate_count(self) -> int:
        return self.recent_start - self.fixed_prefix

    @property
    def fixed_count(self) -> int:
        return self.legal_length - self.candidate_count

    def fixed_positions(self) -> list[int]:
        return [*range(self.fixed_prefix), *range(self.recent_start, self.legal_length)]

    def clamp_k(self, k: int) -> int:
        if k < 0:
            raise ValueError("k must be non-negative")
        return min(int(k), self.candidate_count)

    def selected_count(self, k: int) -> int:
        return self.fixed_count + self.clamp_k(k)


def selection_layout(legal: int, fixed_prefix: int = FIXED_PREFIX, fixed_recent: int = FIXED_RECENT) -> SelectionLayout:
    legal = int(legal)
    if legal < 1:
        raise ValueError("legal length must be positive")
    if fixed_prefix < 0 or fixed_recent < 0:
        raise ValueError("fixed set sizes must be non-negative")
    head = min(int(fixed_prefix), legal)
    tail_start = max(head, legal - int(fixed_recent))
    return SelectionLayout(legal, head, tail_start)


def fixed_budget(n0: int, rho: float, fixed_prefix: int = FIXED_PREFIX, fixed_recent: int = FIXED_RECENT) -> int:
    """k0 of a request whose first decode step has n0 legal positions (round() is Python's ties-to-even)."""
    rho = float(rho)
    if math.isnan(rho) or rho < 0.0 or rho > 1.0:
        raise ValueError("rho must be in [0, 1]")
    candidates = selection_layout(n0, fixed_prefix, fixed_recent).candidate_count
    return min(round(rho * int(n0)), candidates)
