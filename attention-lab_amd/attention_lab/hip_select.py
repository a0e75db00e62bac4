"""Top-k selection on gfx950 (the selection step the reference runs with torch.topk, decode.py:86-93).

Order contract, defined where torch.topk leaves ties unspecified: a larger score ranks first, equal scores rank by the
lower candidate index, NaN ranks below every number, -0.0 equals +0.0. `topk` returns (values, indices) like
torch.topk(..., sorted=True) on the last dimension, for any k in either order; `select_rows` writes the whole row list
of a decode step (F merged with the chosen candidates) in the layout the attend kernel reads.

The tiled kernels' select state and scratch live in a module workspace (or one the caller passes as `workspace=`) that
grows on demand and keeps every buffer it ever handed out alive, so after one eager call of a shape the same calls
allocate nothing and can be captured in a HIP graph, and a later growth never frees memory a captured graph still
uses. Calls that share it must be ordered on one stream (torch's current stream, where every call launches).
"""
from __future__ import annotations

import torch

from . import _native as nat

LDS_SORT_K = nat.LDS_SORT_K   # score order up to this k is sorted in LDS; past it, by a radix pass (tiled entry)
TILED_MIN_M = 32768     # rows at least this long are selected by the tiled kernels (attnlab_topk_tiled)
TILED_MAX_M = 262144    # ... and at most this long (longer rows take the single-workgroup select)
REG_MAX_M = 32768       # rows up to this long fit the single-workgroup select's registers ...
REG_MIN_ROWS = 128      # ... which beats the tiled kernels from this many rows on (the rows alone fill half the chip)
ORDERS = {"position": nat.ORDER_POSITION, "score": nat.ORDER_SCORE}
_WS = nat.Workspace()   # select state (zeroed once, left zeroed by every call) and scratch, per device


def _order_code(order) -> int:
    if order not in ORDERS:
        raise ValueError(f"order must be one of {tuple(ORDERS)}, got {order!r}")
    return ORDERS[order]


def use_tiled(R: int, M: int) -> bool:
    """The automatic choice of topk for R rows of M scores: the tiled kernels for rows of TILED_MIN_M..TILED_MAX_M
    scores, except rows of at most REG_MAX_M scores when there are REG_MIN_ROWS or more of them (one workgroup per
    row, keys in registers). Measured on MI355X at k = M/32, score order: 32K keys, 64 rows: 22.4 us tiled against
    23.8; 256 rows: 33.3 against 27.6; 64K keys, 256 rows: 61.8 tiled against 66.3."""
    return TILED_MIN_M <= M <= TILED_MAX_M and not (M <= REG_MAX_M and R >= REG_MIN_ROWS)


def topk(scores, k: int, *, order: str = "score", tiled=None, workspace=None):
    """Top-k over the last dim of fp32 `scores` [..., M] -> (values fp32 [..., k], indices int64 [..., k]).

    order="score": descending score, ties lowest index first (torch.topk's sorted order with ties defined);
    order="position": the same set, indices ascending. tiled: None picks by use_tiled (and the tiled kernels for
    score order past LDS_SORT_K, which needs their scratch), True / False forces the choice where both apply (same
    result either way).
    """
    if scores.dtype != torch.float32 or not scores.is_cuda:
        raise ValueError("scores must be a float32 tensor on a HIP device")
    if scores.dim() < 1:
        raise ValueError("scores must have at least one dimension")
    code = _order_code(order)
    M = int(scores.shape[-1])
    k = int(k)
    if not 0 <= k <= M:
        raise ValueError(f"need 0 <= k <= {M}, got {k}")
    lead = tuple(scores.shape[:-1])
    s2 = scores.reshape(-1, M)
    if s2.stride(-1) != 1:
        s2 = s2.contiguous()
    R = s2.shape[0]
    idx = torch.empty(R, max(k, 1), dtype=torch.int32, device=scores.device)
    val = torch.empty(R, max(k, 1), dtype=torch.float32, device=scores.device)
    if tiled is None:
        tiled = use_tiled(R, M)
    if code == nat.ORDER_SCORE and k > LDS_SORT_K:
        tiled = True   # the radix pass of a long score order runs in the tiled entry's scratch
    ws = _WS if workspace is None else workspace
    if R and k and tiled:
        state = ws.bytes(scores.device, R * nat.SELECT_STATE_WORDS * 4, "state")
        nbytes = nat.lib().attnlab_select_scratch_bytes(R, M, k, code)
        scratch = ws.bytes(scores.device, nbytes, "scratch")
        nat.call("attnlab_topk_tiled", s2.data_ptr(), s2.stride(0), R, M, k, code, idx.data_ptr(), val.data_ptr(),
                 idx.stride(0), state.data_ptr(), scratch.data_ptr(), scratch.numel(), nat.stream_of(scores.device))
    elif R and k:
        nat.call("attnlab_topk", s2.data_ptr(), s2.stride(0), R, M, k, code, idx.data_ptr(), val.data_ptr(),
                 idx.stride(0), nat.stream_of(scores.device))
    return val[:, :k].reshape(*lead, k), idx[:, :k].long().reshape(*lead, k)


def select_rows(scores, lo: int, hi: int, legal: int, k: int, capacity: int, *, order: str = "position",
                rows=None, want_flat: bool = False, state=None, tiled: bool = True, workspace=None):
    """Row list of one decode step from candidate scores [B, G, hi-lo] (fp32, unit column stride).

    Returns (rows int32 [B, G, S] original positions, flat int64 [B*G*S] row ids of the flattened cache or None),
    S = lo + (legal - hi) + k. order="position" sorts every list ascending (canonical_order); order="score" puts F
    first and then the candidates by descending score, like cat(fixed_rows, topk.indices) in decode.py:93.
    state: the select state score_grouped(..., state=) filled for these scores (cleared here), or None. With a state
    and tiled=True the keys are classified by a grid of 4096-key tiles and each row resolved by one workgroup (same
    result as the single-workgroup select, in either order). Score order takes any k.
    """
    if scores.dim() != 3 or scores.dtype != torch.float32 or not scores.is_cuda or scores.stride(2) != 1:
        raise ValueError("scores must be a float32 [B, G, M] tensor with unit column stride on a HIP device")
    B, G, M = scores.shape
    lo, hi, legal, k, capacity = int(lo), int(hi), int(legal), int(k), int(capacity)
    if M != hi - lo:
        raise ValueError(f"scores hold {M} candidates but hi - lo = {hi - lo}")
    if not 0 <= lo <= hi <= legal <= capacity:
        raise ValueError(f"need 0 <= lo <= hi <= legal <= capacity, got {lo} {hi} {legal} {capacity}")
    if not 0 <= k <= M:
        raise ValueError(f"need 0 <= k <= {M}, got {k}")
    code = _order_code(order)
    S = lo + (legal - hi) + k
    if rows is None:
        rows = torch.empty(B, G, S, dtype=torch.int32, device=scores.device)
    elif rows.dtype != torch.int32 or tuple(rows.shape) != (B, G, S) or not rows.is_contiguous():
        raise ValueError(f"rows must be a contiguous int32 [{B}, {G}, {S}] tensor")
    flat = torch.empty(B * G * S, dtype=torch.int64, device=scores.device) if want_flat else None
    stride = row_stride(scores)
    if stride is None:
        scores = scores.contiguous()
        stride = max(M, 1)
    W = nat.SELECT_STATE_WORDS
    if state is not None and (state.dtype != torch.int32 or tuple(state.shape) != (B, G, W)
                              or not state.is_contiguous() or state.device != scores.device):
        raise ValueError(f"state must be a contiguous int32 [{B}, {G}, {W}] tensor on the scores' device")
    scratch = None
    if k > 0 and ((state is not None and tiled) or (code == nat.ORDER_SCORE and k > LDS_SORT_K)):
        nbytes = nat.lib().attnlab_select_scratch_bytes(B * G, M, k, code)
        scratch = (_WS if workspace is None else workspace).bytes(scores.device, nbytes, "scratch")
    nat.call("attnlab_select_rows", scores.data_ptr(), stride, B, G, lo, hi, legal, k, capacity, code,
             rows.data_ptr(), S, nat.ptr(flat), nat.ptr(state), nat.ptr(scratch),
             0 if scratch is None else scratch.numel(), nat.stream_of(scores.device))
    return rows, flat


def row_stride(t3):
    """Stride s such that row (b, g) of a [B, G, M] tensor starts at element (b*G + g) * s, or None."""
    B, G, M = t3.shape
    if t3.stride(2) != 1 and M > 1:
        return None
    if B * G == 1:
        return max(M, 1)
    s = t3.stride(1) if G > 1 else t3.stride(0)
    if B > 1 and t3.stride(0) != G * s:
        return None
    return s if s >= M else None
