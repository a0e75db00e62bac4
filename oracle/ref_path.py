"""The reference's own op sequence for one decode step, on the CPU with torch. Test infrastructure only.

This is what the reference executes per layer and step (decode.py:145-163 -> indexer.py:15-29, decode.py:86-93,
131-142, sparse.py:40-60; dense: full.py:17-34): bmm + strided column copy for z, bmm for u, bmm over the candidate
columns, torch.topk, cat with the fixed rows, two flattened index_selects, SDPA with the h heads folded into the
sequence axis. bench.py times it on the host cores as the CPU baseline; tests compare it with `exact`.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import rules


def sparse_layer_step(q_main, q_pre, k_cache, v_cache, zT, wq_t_scaled, wk, k_pre_new, legal: int, k0: int,
                      scale=None):
    """q_main/q_pre [B,G,h,1,d]; caches [B,G,C,d]; zT [B,G,r,C] (column legal-1 is written); returns (out, rows)."""
    B, G, h, T, d = q_main.shape
    C = k_cache.shape[2]
    lo, hi, k, S = rules.step(legal, k0)
    wc = legal - 1
    zT[..., wc:wc + 1].copy_(torch.matmul(wk.unsqueeze(0), k_pre_new.transpose(-1, -2)))
    q_cat = q_pre.permute(0, 1, 3, 2, 4).reshape(B, G, T, h * d)
    u = torch.matmul(q_cat, wq_t_scaled.unsqueeze(0))
    offsets = (torch.arange(B * G, dtype=torch.long) * C).view(B, G, 1)
    fixed = torch.tensor(rules.fixed_positions(legal), dtype=torch.long).view(1, 1, -1) + offsets
    if k > 0:
        scores = torch.matmul(u, zT[..., lo:hi])
        top = torch.topk(scores, k, dim=-1).indices.view(B, G, k)
        rows = torch.cat([fixed, top + offsets + lo], dim=-1).reshape(-1)
    else:
        rows = fixed.reshape(-1)
    k_sub = k_cache.reshape(B * G * C, d).index_select(0, rows).view(B, G, S, d)
    v_sub = v_cache.reshape(B * G * C, d).index_select(0, rows).view(B, G, S, d)
    out = F.scaled_dot_product_attention(q_main.reshape(B, G, h * T, d), k_sub, v_sub, scale=scale)
    return out.view(B, G, h, T, d), rows


def dense_layer_step(q_main, k_cache, v_cache, legal: int, scale=None):
    """full_attention(backend="sdpa_fold") for one query at position legal-1 (full.py:31-34): no mask."""
    B, G, h, T, d = q_main.shape
    out = F.scaled_dot_product_attention(q_main.reshape(B, G, h * T, d), k_cache[:, :, :legal], v_cache[:, :, :legal],
                                         scale=scale)
    return out.view(B, G, h, T, d)
