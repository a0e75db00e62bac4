"""Row addressing of the static cache and the gather-free subset read.

Same names as the reference's sparse module (src/attention_lab/sparse.py:14-67). The reference reads a subset by
materialising it (index_select of K and V rows, then SDPA over the copies); here `gather_attention` hands the
position list to the attend kernel, which reads each listed K/V row straight from the cache. `gather_rows` is kept as
a data-movement utility (the reference's tests use it to check that positions are original), and `subset_attention`
attends over such an already gathered subset on the same kernel (its rows are the subset's own slots).
"""
from __future__ import annotations

import torch

from . import hip_attend


def row_offsets(batch: int, groups: int, capacity: int, device) -> torch.Tensor:
    """[B,G,1] int64 offsets that turn a position into a row id of the flattened [B*G*C, d] cache."""
    return (torch.arange(batch * groups, device=device, dtype=torch.long) * capacity).view(batch, groups, 1)


def flatten_cache(x: torch.Tensor) -> torch.Tensor:
    """[B,G,C,d] contiguous -> [B*G*C, d] view. Never copies: raises instead."""
    if x.dim() != 4:
        raise ValueError(f"cache must be [B,G,C,d], got {tuple(x.shape)}")
    if not x.is_contiguous():
        raise ValueError("cache must be contiguous so the flattened view is free")
    B, G, C, d = x.shape
    return x.view(B * G * C, d)


def gather_rows(x: torch.Tensor, selected: torch.Tensor, offsets=None) -> torch.Tensor:
    """x [B,G,C,d], selected [B,G,S] original positions -> copies [B,G,S,d] (row s of (b,g) is x[b,g,selected[b,g,s]])."""
    B, G, C, d = x.shape
    if selected.dim() != 3 or tuple(selected.shape[:2]) != (B, G):
        raise ValueError(f"selected must be [B,G,S] matching the cache, got {tuple(selected.shape)}")
    S = selected.shape[-1]
    off = row_offsets(B, G, C, x.device) if offsets is None else offsets
    return flatten_cache(x).index_select(0, (selected + off).reshape(-1)).view(B, G, S, d)


def gather_attention(q, k, v, selected, selected_valid=None, *, scale=None, backend="sdpa", offsets=None):
    """Attention of q [B,G,h,1,d] over the listed original positions selected [B,G,S], read in place.

    Padded slots (selected_valid False) become position -1, which the kernel skips. `offsets` is accepted for
    signature compatibility; positions are always relative to their own (b, g) block.
    """
    if backend not in ("sdpa", "explicit"):
        raise ValueError(f"unknown subset backend {backend!r}")
    B, G, h, T, d = q.shape
    if T != 1:
        raise ValueError("the gather-free read takes one query position")
    pos = selected if selected_valid is None else torch.where(selected_valid, selected, torch.full_like(selected, -1))
    pos = pos.to(torch.int32).contiguous()
    out = hip_attend.attend(q.reshape(B, G, h, d).contiguous(), k, v, pos, scale=scale, out_dtype=q.dtype)
    return out.view(B, G, h, 1, d)


def subset_attention(q, k_sub, v_sub, valid_mask=None, *, scale=None, backend="sdpa"):
    """Attention of q [B,G,h,T,d] over a gathered subset k_sub, v_sub [B,G,S,d] -> [B,G,h,T,d] (sparse.py:40-60).

    The h*T query rows of a group share the S subset rows (each row is read once per group), so the T queries fold
    into the head axis of the attend kernel. valid_mask [B,G,S] (bool) drops padded slots; a group with no valid slot
    has no defined output.

    Narrower than the reference, which takes any dtype and head dim through torch: this runs only on the HIP attend
    kernel, so q, k_sub and v_sub must be bfloat16 on a HIP device with d = 128 and h*T <= 8 query rows per group;
    other inputs raise ValueError naming the restriction (there is no torch fallback). Both backend names run that
    one kernel: "sdpa" and "explicit" compute the same softmax attention and differ only in rounding in the
    reference, and the kernel accumulates in fp32 either way.
    """
    if backend not in ("sdpa", "explicit"):
        raise ValueError(f"unknown subset backend {backend!r}")
    if q.dim() != 5 or k_sub.dim() != 4 or v_sub.shape != k_sub.shape:
        raise ValueError("q must be [B,G,h,T,d] and k_sub, v_sub [B,G,S,d]")
    B, G, h, T, d = q.shape
    S = int(k_sub.shape[2])
    if tuple(k_sub.shape[:2]) != (B, G) or k_sub.shape[3] != d:
        raise ValueError(f"subset {tuple(k_sub.shape)} does not match q {tuple(q.shape)}")
    for t, n in ((q, "q"), (k_sub, "k_sub"), (v_sub, "v_sub")):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"subset_attention on the HIP attend kernel takes bfloat16 only; {n} is {t.dtype}")
    if d != hip_attend.HEAD_DIM:
        raise ValueError(f"subset_attention on the HIP attend kernel takes head_dim {hip_attend.HEAD_DIM} only, got {d}")
    if h * T > hip_attend.MAX_H:
        raise ValueError(f"subset_attention on the HIP attend kernel takes h*T <= {hip_attend.MAX_H} query rows per "
                         f"group, got {h * T}")
    slots = torch.arange(S, device=k_sub.device, dtype=torch.int32).expand(B, G, S)
    if valid_mask is not None:
        if tuple(valid_mask.shape) != (B, G, S):
            raise ValueError(f"valid_mask must be [B,G,S] = [{B},{G},{S}]")
        slots = torch.where(valid_mask.bool(), slots, torch.full_like(slots, -1))
    qf = q.reshape(B, G, h * T, d).contiguous()
    out = hip_attend.attend(qf, k_sub.contiguous(), v_sub.contiguous(), slots.contiguous(), scale=scale,
                            out_dtype=q.dtype)
    return out.view(B, G, h, T, d)
