"""Full attention A over every legal position, on the dense decode kernel.

Same signature and validation as the reference's full_attention (src/attention_lab/full.py:14-44). Every backend
name of the reference is accepted; all of them read K and V once per KV group (the reference's sdpa_fold
behaviour), which is the only layout the HIP kernel has. A single query at the last legal position needs no mask
(full.py:29). Several queries (a prefill chunk) follow the reference's legality rule (reference.py:41-48: key j is
legal for query t iff j <= its position and j < valid_length). Consecutive positions (a prefill chunk) run the causal
prefill kernel on the matrix cores in one launch; any other position list runs one dense-decode launch per query
over the first min(position_t + 1, valid_length) positions.
"""
from __future__ import annotations

import torch

from . import hip_attend

FULL_BACKENDS = ("sdpa_fold", "sdpa_gqa", "sdpa_repeat", "explicit")


def _check_shapes(q, k, v):
    if q.dim() != 5:
        raise ValueError(f"q must be [B,G,h,T,d], got {tuple(q.shape)}")
    if k.dim() != 4 or v.dim() != 4:
        raise ValueError(f"k and v must be [B,G,C,d], got {tuple(k.shape)} and {tuple(v.shape)}")
    B, G, h, T, d = q.shape
    if k.shape[0] != B or k.shape[1] != G or k.shape[3] != d or v.shape != k.shape:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    return B, G, h, T, d, k.shape[2]


def full_attention(q, k, v, *, valid_length=None, query_positions=None, scale=None, backend="sdpa_fold"):
    """q [B,G,h,T,d]; k, v [B,G,C,d]; reads k[:, :, :valid_length]. Returns [B,G,h,T,d]."""
    B, G, h, T, d, C = _check_shapes(q, k, v)
    legal = C if valid_length is None else int(valid_length)
    if not 0 < legal <= C:
        raise ValueError(f"valid_length={legal} must be in (0, capacity={C}]")
    if backend not in FULL_BACKENDS:
        raise ValueError(f"unknown full-attention backend {backend!r}; choose from {FULL_BACKENDS}")
    # default: the T queries sit at the last T legal positions (reference.py:114-118)
    qp = list(range(legal - T, legal)) if query_positions is None else [int(p) for p in query_positions]
    if len(qp) != T:
        raise ValueError(f"need {T} query positions, got {len(qp)}")
    if min(qp) < 0:
        raise ValueError("query positions must be non-negative")
    if T == 1 and qp[0] >= legal - 1:
        out = hip_attend.dense_decode(q.reshape(B, G, h, d).contiguous(), k, v, legal, scale=scale, out_dtype=q.dtype)
        return out.view(B, G, h, 1, d)
    if (q.dtype == torch.bfloat16 and h in hip_attend.PREFILL_HEADS and d == hip_attend.HEAD_DIM
            and qp == list(range(qp[0], qp[0] + T))):
        # consecutive positions (a prefill chunk): one launch of the causal prefill kernel
        return hip_attend.prefill_attend(q.contiguous(), k, v, qp[0], legal, scale=scale)
    out = torch.empty(B, G, h, T, d, dtype=q.dtype, device=q.device)
    for t, p in enumerate(qp):
        out[:, :, :, t] = hip_attend.dense_decode(q[:, :, :, t].contiguous(), k, v, min(p + 1, legal), scale=scale,
                                                  out_dtype=q.dtype)
    return out
