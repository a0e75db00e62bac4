"""Grouped indexer: one (Wq, Wk) pair per KV group; u = Wq.concat_h(q_pre)/sqrt(r), z = Wk.k_pre, score = u.z.

Same construction and names as the reference (src/attention_lab/indexer.py:15-64): the index keys live transposed as
zT [B,G,r,C] so a decode step scans the contiguous slice zT[..., lo:hi]; `GroupedIndexer` draws its weights with
the same seeded float64 generator calls (wq first, then wk, both scaled by init_std), so a given seed yields the
reference's weights bit for bit, and 1/sqrt(r) is folded into wq_t_scaled. The projections and the scan run on the
HIP kernels (bfloat16 tables and weights).
"""
from __future__ import annotations

import math

import torch

from . import _native as nat
from .hip_score import candidate_scores, project_queries

__all__ = ["GroupedIndexer", "candidate_scores", "project_keys", "project_queries"]


def project_keys(k_pre: torch.Tensor, wk: torch.Tensor, *, out=None, col0: int = 0) -> torch.Tensor:
    """k_pre [B,G,T,d], wk [G,r,d] -> zT [B,G,r,T] (or written into out[..., col0:col0+T] of a [B,G,r,C] table)."""
    if k_pre.dim() != 4 or wk.dim() != 3:
        raise ValueError("k_pre must be [B,G,T,d] and wk [G,r,d]")
    B, G, T, d = k_pre.shape
    if wk.shape[0] != G or wk.shape[2] != d:
        raise ValueError(f"wk {tuple(wk.shape)} does not match k_pre {tuple(k_pre.shape)}")
    dt = wk.dtype
    if dt not in (torch.bfloat16, torch.float32) or k_pre.dtype != dt or not k_pre.is_cuda or wk.device != k_pre.device:
        raise ValueError("k_pre and wk must both be bfloat16 (or both float32, a trained bank) on one HIP device")
    align = 8 if dt == torch.bfloat16 else 4   # elements per 16 bytes
    r = int(wk.shape[1])
    bg_stride = k_pre.stride(1) if G > 1 else k_pre.stride(0)
    strided_ok = (k_pre.stride(3) == 1 and (B == 1 or k_pre.stride(0) == G * bg_stride) and bg_stride % align == 0
                  and k_pre.stride(2) % align == 0 and k_pre.data_ptr() % 16 == 0)
    if not strided_ok:
        k_pre = k_pre.contiguous()
        bg_stride = T * d
    if out is None:
        out = torch.empty(B, G, r, T, dtype=dt, device=k_pre.device)
        col0 = 0
    elif out.dim() != 4 or tuple(out.shape[:3]) != (B, G, r) or out.dtype != dt or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous {dt} [{B}, {G}, {r}, C] table")
    wkc = wk.contiguous()
    entry = "attnlab_project_keys" if dt == torch.bfloat16 else "attnlab_project_keys_f32"
    nat.call(entry, k_pre.data_ptr(), bg_stride, k_pre.stride(2), wkc.data_ptr(), out.data_ptr(), B, G, T, r, d,
             int(out.shape[3]), int(col0), nat.stream_of(k_pre.device))
    return out


class GroupedIndexer:
    """Untrained random indexer for one layer (weights ~ init_std * N(0, 1), drawn in float64 on the CPU)."""

    def __init__(self, groups: int, heads_per_group: int, head_dim: int, r: int = 32, *, device="cpu",
                 dtype=torch.float32, seed: int = 0, init_std: float = 0.02):
        self.groups, self.heads_per_group, self.head_dim, self.r = int(groups), int(heads_per_group), int(head_dim), int(r)
        gen = torch.Generator().manual_seed(int(seed))
        wq = torch.randn(self.groups, self.r, self.heads_per_group * self.head_dim, generator=gen, dtype=torch.float64)
        wk = torch.randn(self.groups, self.r, self.head_dim, generator=gen, dtype=torch.float64)
        wq, wk = wq * init_std, wk * init_std
        self.wq = wq.to(device=device, dtype=dtype)                                    # [G, r, h*d], unscaled
        self.wk = wk.to(device=device, dtype=dtype)                                    # [G, r, d]
        self.wq_t_scaled = (wq / math.sqrt(self.r)).transpose(1, 2).contiguous().to(device=device, dtype=dtype)

    def keys(self, k_pre: torch.Tensor) -> torch.Tensor:
        """[B,G,T,d] -> [B,G,r,T] index keys (a chunk of the transposed table)."""
        return project_keys(k_pre, self.wk)

    def query(self, q_pre: torch.Tensor) -> torch.Tensor:
        return project_queries(q_pre, self.wq_t_scaled)

    def scores(self, u: torch.Tensor, zT: torch.Tensor, lo: int = 0, hi=None) -> torch.Tensor:
        return candidate_scores(u, zT, lo, zT.shape[-1] if hi is None else hi)

    def reference_scores(self, q_pre: torch.Tensor, k_pre: torch.Tensor, lo: int = 0, hi=None) -> torch.Tensor:
        """float64 CPU brute force from the stored weights (indexer.py:57-64): scores [B,G,T,hi-lo] of the T queries
        q_pre [B,G,h,T,d] against the keys k_pre [B,G,C,d], (wq . concat_h q)(wk . k) / sqrt(r) over [lo, hi)."""
        B, G, h, T, d = q_pre.shape
        hi = int(k_pre.shape[2]) if hi is None else int(hi)
        q_cat = q_pre.detach().double().cpu().permute(0, 1, 3, 2, 4).reshape(B, G, T, h * d)
        u = torch.einsum("bgtf,grf->bgtr", q_cat, self.wq.detach().double().cpu())
        z = torch.einsum("grd,bgcd->bgrc", self.wk.detach().double().cpu(), k_pre.detach().double().cpu()[:, :, lo:hi])
        return torch.einsum("bgtr,bgrc->bgtc", u, z) / math.sqrt(self.r)
