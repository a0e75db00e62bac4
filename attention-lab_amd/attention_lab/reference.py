"""Explicit attention references: the comparison targets the reference package exports (src/attention_lab/reference.py:
41-97), written out as scores -> mask -> softmax -> weighted sum. They are not a compute path of this package (the
reads run on the HIP kernels in full.py / sparse.py / decode.py) and nothing here is called by them.

The arithmetic runs in float32 (float64 inputs stay float64) on the inputs' device and the result is returned in q's
dtype, so a bfloat16 check never goes through a bfloat16 batched product. Shapes: q [B,G,h,T,d]; k, v [B,G,C,d];
selected [B,G,S] positions; output [B,G,h,T,d].
"""
from __future__ import annotations

import math

import torch

__all__ = ["dense_reference", "dense_mask_reference", "legality_mask", "selection_mask"]


def _dims(q, k, v):
    if q.dim() != 5:
        raise ValueError(f"q must be [B,G,h,T,d], got {tuple(q.shape)}")
    if k.dim() != 4 or v.dim() != 4:
        raise ValueError(f"k and v must be [B,G,C,d], got {tuple(k.shape)} and {tuple(v.shape)}")
    B, G, h, T, d = q.shape
    if (k.shape[0], k.shape[1], k.shape[3]) != (B, G, d) or v.shape != k.shape:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    return B, G, h, T, d, int(k.shape[2])


def _legal(valid_length, C):
    n = C if valid_length is None else int(valid_length)
    if not 0 < n <= C:
        raise ValueError(f"valid_length={n} must be in (0, capacity={C}]")
    return n


def _work_dtype(t):
    return torch.float64 if t.dtype == torch.float64 else torch.float32


def legality_mask(query_positions, legal: int, device) -> torch.Tensor:
    """[T, legal] bool: key j is visible to the query at position p iff j <= p (j < legal by construction)."""
    pos = torch.as_tensor([int(p) for p in query_positions], dtype=torch.long, device=device)
    mask = torch.arange(legal, device=device).unsqueeze(0) <= pos.unsqueeze(1)
    if not bool(mask.any(dim=1).all()):
        raise ValueError("a query has no legal key position")
    return mask


def selection_mask(selected, legal: int, selected_valid=None) -> torch.Tensor:
    """[B,G,legal] bool from a position list [B,G,S]; slots with selected_valid False are dropped."""
    if selected.dim() != 3 or selected.dtype not in (torch.int32, torch.int64):
        raise ValueError("selected must be an integer tensor [B,G,S]")
    if selected.numel() and (int(selected.min()) < 0 or int(selected.max()) >= legal):
        raise ValueError(f"selected positions must lie in [0, {legal})")
    B, G, _ = selected.shape
    keep = torch.zeros(B, G, legal, dtype=torch.bool, device=selected.device)
    pos = selected.long()
    if selected_valid is not None:
        pos = torch.where(selected_valid.bool(), pos, torch.full_like(pos, legal))   # dropped slots -> a spare column
        keep = torch.zeros(B, G, legal + 1, dtype=torch.bool, device=selected.device)
    keep.scatter_(2, pos, True)
    return keep[..., :legal]


def _attend(q, k, v, allow, scale):
    """softmax over the allowed columns of scale * q.k, then the weighted sum of v; allow [B,G,1|h,T,L] bool."""
    wt = _work_dtype(q)
    qf, kf, vf = q.to(wt), k.to(wt), v.to(wt)
    s = torch.einsum("bgitd,bgld->bgitl", qf, kf) * scale
    s = s.masked_fill(~allow, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.einsum("bgitl,bgld->bgitd", p, vf).to(q.dtype)


def dense_reference(q, k, v, *, valid_length=None, query_positions=None, scale=None):
    """Every legal key, causally masked by query position (default: the T queries are the last T legal positions)."""
    B, G, h, T, d, C = _dims(q, k, v)
    legal = _legal(valid_length, C)
    qp = list(range(legal - T, legal)) if query_positions is None else [int(p) for p in query_positions]
    if len(qp) != T:
        raise ValueError(f"need {T} query positions, got {len(qp)}")
    if min(qp) < 0:
        raise ValueError("query positions must be non-negative")
    sc = 1.0 / math.sqrt(d) if scale is None else float(scale)
    allow = legality_mask(qp, legal, q.device).view(1, 1, 1, T, legal)
    return _attend(q, k[:, :, :legal], v[:, :, :legal], allow, sc)


def dense_mask_reference(q, k, v, selected, selected_valid=None, *, valid_length=None, scale=None):
    """Attention restricted to the listed positions (shared by the h*T queries of a group): all legal scores, every
    column outside the list masked."""
    B, G, h, T, d, C = _dims(q, k, v)
    legal = _legal(valid_length, C)
    keep = selection_mask(selected, legal, selected_valid)
    if not bool(keep.any(dim=-1).all()):
        raise ValueError("empty selection for some (batch, group)")
    sc = 1.0 / math.sqrt(d) if scale is None else float(scale)
    return _attend(q, k[:, :, :legal], v[:, :, :legal], keep.view(B, G, 1, 1, legal), sc)
