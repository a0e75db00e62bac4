"""One decode step of one layer: the dense read (A) and the index-selected read (D), on HIP kernels.

Public names, arguments and shapes follow the reference's decode module (src/attention_lab/decode.py:26-176) so the
module is a drop-in for it; the torch ops under each function are replaced by the gfx950 kernels:

* `sparse_decode_step_kernel` - z column write + u projection + candidate scan (one launch), top-k + merge with F
  (one launch), gather-free attention (one launch with in-kernel split-K merge). The reference runs about ten torch
  ops here (docs/SCOPING_FUSED_D_KERNEL.md:9-24).
* `select_rows_kernel` - candidate scan from a given u, then the select kernel writing flat row ids in the
  reference's order (F first, then the candidates by descending score).
* `gathered_decode_step_kernel` - the attend kernel on a given flat row list.
* `dense_decode_step` - the dense decode kernel.

The `backend` arguments are validated as in the reference and otherwise ignored: the HIP kernels are the backend.
The selection tie order is defined (equal scores: lower position first) where torch.topk leaves it open. Only
bfloat16 K/V caches with head_dim 128 and T == 1 run here, over a bfloat16 index table or a trained bank's float32
one (trained.py:78-81); other inputs raise ValueError.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _native as nat
from . import hip_attend, hip_score, hip_select
from .indexer import GroupedIndexer
from .selection import FIXED_PREFIX, FIXED_RECENT, SelectionLayout, fixed_budget, legal_length, selection_layout
from .sparse import flatten_cache, row_offsets

SUBSET_BACKENDS = ("sdpa", "explicit")


@dataclass
class DecodeRequest:
    """Per-request constants for one legal length: layout, budget and the fixed set's positions and row ids."""

    layout: SelectionLayout
    k0: int
    k: int
    batch: int
    groups: int
    capacity: int
    offsets: torch.Tensor          # [B,G,1] row offsets into the flattened [B*G*C, d] cache
    fixed_positions: torch.Tensor  # [B,G,F] original positions of F
    fixed_rows: torch.Tensor       # [B,G,F] = fixed_positions + offsets
    off_lo: torch.Tensor           # [B,G,1] = offsets + candidate_lo

    @property
    def selected_count(self) -> int:
        return self.layout.fixed_count + self.k

    @property
    def write_col(self) -> int:
        """Index-table column of the newest key (the query's own position)."""
        return self.layout.legal_length - 1

    def topk_candidates(self, u: torch.Tensor, zT: torch.Tensor) -> torch.Tensor:
        """[B,G,k] candidate-relative indices, descending score (ties: lower index first)."""
        if self.k <= 0:
            return torch.empty(self.batch, self.groups, 0, dtype=torch.long, device=u.device)
        s = hip_score.candidate_scores(u, zT, self.layout.candidate_lo, self.layout.candidate_hi)
        return hip_select.topk(s.view(self.batch, self.groups, -1), self.k, order="score")[1]

    def select_positions(self, u: torch.Tensor, zT: torch.Tensor) -> torch.Tensor:
        """[B,G,S] original positions: F first, then the chosen candidates."""
        top = self.topk_candidates(u, zT) + self.layout.candidate_lo
        return torch.cat([self.fixed_positions, top], dim=-1)

    def select_rows(self, u: torch.Tensor, zT: torch.Tensor) -> torch.Tensor:
        """Flat row ids [B*G*S] of the flattened cache."""
        return select_rows_kernel(u, zT, self.fixed_rows, self.off_lo, self.layout.candidate_lo,
                                  self.layout.candidate_hi, self.k)


F_TAG = "_attnlab_standard_f"   # attribute set on fixed_rows / off_lo tensors built by the selection rule here


def tag_standard_f(fixed_rows: torch.Tensor, off_lo: torch.Tensor, lo: int, hi: int, legal: int, capacity: int):
    """Mark (fixed_rows, off_lo) as the rule's F of (lo, hi, legal) in a cache of `capacity` rows per (b, g), so the
    HIP steps accept them without comparing their values on the device."""
    key = (int(lo), int(hi), int(legal), int(capacity))
    setattr(fixed_rows, F_TAG, key)
    setattr(off_lo, F_TAG, key)
    return fixed_rows, off_lo


def check_standard_f(fixed_rows, off_lo, lo: int, hi: int, legal: int, capacity: int) -> None:
    """The HIP step writes F itself from (lo, hi, legal) (its row list is F = [0, lo) U [hi, legal) then the top-k),
    where the reference concatenates the fixed_rows it is given (decode.py:86-93). Every caller of the reference passes
    the rule's F (decode.py:179-194, qwen_wrap.py:169-181); anything else is refused rather than silently replaced.
    Tensors tagged by tag_standard_f pass without a device read; others are compared on the device (one sync)."""
    key = (int(lo), int(hi), int(legal), int(capacity))
    if getattr(fixed_rows, F_TAG, None) == key and getattr(off_lo, F_TAG, None) == key:
        return
    B, G = int(fixed_rows.shape[0]), int(fixed_rows.shape[1])
    offsets = row_offsets(B, G, capacity, fixed_rows.device)
    pos = torch.tensor(list(range(lo)) + list(range(hi, legal)), dtype=torch.long, device=fixed_rows.device)
    want = pos.view(1, 1, -1) + offsets
    if (tuple(fixed_rows.shape) != tuple(want.shape) or not torch.equal(fixed_rows.long(), want)
            or not torch.equal(off_lo.long(), offsets + lo)):
        raise ValueError("fixed_rows / off_lo must hold the selection rule's F = [0, lo) U [hi, legal) plus the row "
                         "offsets (b*G + g)*C: the HIP step writes F from (lo, hi, legal) and cannot read another set")


def prepare_request(batch: int, groups: int, capacity: int, *, valid_length: int, query_position: int, rho: float,
                    device, n0=None, fixed_prefix: int = FIXED_PREFIX, fixed_recent: int = FIXED_RECENT) -> DecodeRequest:
    """Fix k0 from the request's starting length n0 (default: the current legal length); clamp k to this step."""
    legal = legal_length(query_position, valid_length)
    if legal > capacity:
        raise ValueError(f"legal length {legal} exceeds allocated capacity {capacity}")
    k0 = fixed_budget(legal if n0 is None else int(n0), rho, fixed_prefix, fixed_recent)
    layout = selection_layout(legal, fixed_prefix, fixed_recent)
    k = layout.clamp_k(k0)
    offsets = row_offsets(batch, groups, capacity, device)
    fixed = torch.tensor(layout.fixed_positions(), dtype=torch.long, device=device)
    fixed = fixed.view(1, 1, -1).expand(batch, groups, -1).contiguous()
    fixed_rows, off_lo = tag_standard_f((fixed + offsets).contiguous(), (offsets + layout.candidate_lo).contiguous(),
                                        layout.candidate_lo, layout.candidate_hi, legal, capacity)
    return DecodeRequest(layout=layout, k0=k0, k=k, batch=batch, groups=groups, capacity=capacity, offsets=offsets,
                         fixed_positions=fixed, fixed_rows=fixed_rows, off_lo=off_lo)


def _layout_from_rows(fixed_rows, lo: int, hi: int, k: int, selected_count: int):
    """Recover legal from the reference's (fixed_rows, lo, hi, k, S) arguments: F = [0, lo) U [hi, legal)."""
    nf = int(fixed_rows.shape[-1])
    if selected_count != nf + k:
        raise ValueError(f"selected_count={selected_count} != |F| + k = {nf} + {k}")
    legal = hi + (nf - lo)
    if lo < 0 or hi < lo or legal < hi:
        raise ValueError(f"fixed set of {nf} rows does not match the candidate domain [{lo}, {hi})")
    return legal


def _order(canonical_order: bool) -> str:
    return "position" if canonical_order else "score"


def select_rows_kernel(u, zT, fixed_rows, off_lo, lo: int, hi: int, k: int) -> torch.Tensor:
    """D0: score the candidate columns from u, one top-k, merge with F. Returns flat int64 row ids [B*G*S].

    The kernel writes F from (lo, hi, legal); fixed_rows / off_lo must be the rule's F and offsets (check_standard_f).
    """
    B, G = fixed_rows.shape[:2]
    C = int(zT.shape[-1])
    if k <= 0:
        return fixed_rows.reshape(-1)
    legal = _layout_from_rows(fixed_rows, lo, hi, k, int(fixed_rows.shape[-1]) + k)
    check_standard_f(fixed_rows, off_lo, lo, hi, legal, C)
    s = hip_score.candidate_scores(u, zT, lo, hi).view(B, G, hi - lo)
    _, flat = hip_select.select_rows(s, lo, hi, legal, k, C, order="score", want_flat=True)
    return flat


def select_rows_recent(fixed_rows, off_lo, lo: int, hi: int, k: int) -> torch.Tensor:
    """B selector (reference decode.py:96-109): the k most recent candidates [hi - k, hi) after F, as flat row ids.

    Candidate-relative index i maps to row off_lo + i, as the top-k indices of the index selector do; nothing is scored.
    """
    B, G = fixed_rows.shape[:2]
    if k <= 0:
        return fixed_rows.reshape(-1)
    M = hi - lo
    if k > M:
        raise ValueError(f"k={k} exceeds the candidate count {M}")
    rel = torch.arange(M - k, M, device=fixed_rows.device, dtype=torch.long).expand(B, G, k)
    return torch.cat([fixed_rows, rel + off_lo], dim=-1).reshape(-1)


def select_rows_uniform(fixed_rows, off_lo, lo: int, hi: int, k: int, *, rng) -> torch.Tensor:
    """C selector (reference decode.py:112-128): k candidates drawn uniformly without replacement per (b, g), after F.

    `rng` is a numpy Generator; the draw is the top k of B*G*M float64 uniforms taken from it in one call, so a given
    generator state yields the reference's rows. Not a learned choice.
    """
    import numpy as np   # the package stays importable without numpy
    B, G = fixed_rows.shape[:2]
    if k <= 0:
        return fixed_rows.reshape(-1)
    M = hi - lo
    if k > M:
        raise ValueError(f"k={k} exceeds the candidate count {M}")
    draws = torch.from_numpy(rng.random((B, G, M), dtype=np.float64))
    rel = torch.topk(draws, k, dim=-1).indices.to(fixed_rows.device)
    return torch.cat([fixed_rows, rel + off_lo], dim=-1).reshape(-1)


def _positions_from_flat(rows, B, G, S, C, device):
    off = row_offsets(B, G, C, device)
    pos = rows.view(B, G, S) - off
    return pos.to(torch.int32).contiguous()


def gathered_decode_step_kernel(q_main, k_cache, v_cache, rows, selected_count: int, *, scale=None, backend="sdpa"):
    """Read exactly the listed rows (flat ids into the flattened [B*G*C, d] cache) and attend over them."""
    if backend not in SUBSET_BACKENDS:
        raise ValueError(f"unknown subset backend {backend!r}")
    B, G, h, T, d = q_main.shape
    if T != 1:
        raise ValueError("a decode step takes exactly one new query position")
    flatten_cache(k_cache)
    flatten_cache(v_cache)
    C = int(k_cache.shape[2])
    pos = _positions_from_flat(rows, B, G, selected_count, C, k_cache.device)
    q = q_main.reshape(B, G, h, d).contiguous()
    out = hip_attend.attend(q, k_cache, v_cache, pos, scale=scale, out_dtype=q_main.dtype)
    return out.view(B, G, h, 1, d)


_STEP_WS = nat.Workspace()   # scores / row list / partials and the select state of sparse_decode_step_kernel


def sparse_decode_step_kernel(q_main, q_pre, k_cache, v_cache, zT, wq_t_scaled, wk, fixed_rows, off_lo, lo: int,
                              hi: int, k: int, selected_count: int, *, k_pre_new=None, write_col: int = -1,
                              scale=None, backend="sdpa", return_rows: bool = False, canonical_order: bool = False,
                              partitions=None, workspace=None):
    """One layer's D read for one new query (T == 1) as three HIP launches; same contract as decode.py:145-163.

    `return_rows=True` also returns the flat row ids that were read. canonical_order=True lists every row set in
    ascending position; otherwise F comes first and the candidates follow by descending score. `workspace` (a
    _native.Workspace; default: one shared by the module) holds the step's scratch and select state; see Workspace
    for HIP graph capture.
    """
    if backend not in SUBSET_BACKENDS:
        raise ValueError(f"unknown subset backend {backend!r}")
    B, G, h, T, d = q_main.shape
    if T != 1:
        raise ValueError("a decode step takes exactly one new query position")
    # the index side is bfloat16, or float32 throughout for a trained bank (trained.py:78-81)
    idx_dt = zT.dtype
    if idx_dt not in (torch.bfloat16, torch.float32):
        raise ValueError(f"zT must be bfloat16 or float32, got {idx_dt}")
    for t, n, want in ((q_main, "q_main", torch.bfloat16), (q_pre, "q_pre", idx_dt), (k_cache, "k_cache", torch.bfloat16),
                       (v_cache, "v_cache", torch.bfloat16), (zT, "zT", idx_dt), (wq_t_scaled, "wq_t_scaled", idx_dt),
                       (wk, "wk", idx_dt)):
        if t.dtype != want:
            raise ValueError(f"{n} must be {want} on the HIP path, got {t.dtype}")
        if not t.is_cuda:
            raise ValueError(f"{n} must live on a HIP device")
    if d != hip_attend.HEAD_DIM or not 1 <= h <= hip_attend.MAX_H:
        raise ValueError(f"the HIP path needs head_dim {hip_attend.HEAD_DIM} and 1 <= h <= {hip_attend.MAX_H}")
    flatten_cache(k_cache)
    flatten_cache(v_cache)
    Bc, Gc, C, dc = k_cache.shape
    if (Bc, Gc, dc) != (B, G, d) or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache/v_cache must be [B, G, C, d] matching q_main")
    if zT.dim() != 4 or tuple(zT.shape[:2]) != (B, G) or zT.shape[3] != C or not zT.is_contiguous():
        raise ValueError("zT must be a contiguous [B, G, r, C] tensor matching the cache")
    r = int(zT.shape[2])
    if tuple(wq_t_scaled.shape) != (G, h * d, r) or tuple(wk.shape) != (G, r, d):
        raise ValueError("wq_t_scaled must be [G, h*d, r] and wk [G, r, d]")
    if tuple(fixed_rows.shape[:2]) != (B, G) or tuple(off_lo.shape) != (B, G, 1):
        raise ValueError("fixed_rows must be [B, G, F] and off_lo [B, G, 1]")
    lo, hi, k, S = int(lo), int(hi), int(k), int(selected_count)
    legal = _layout_from_rows(fixed_rows, lo, hi, k, S)
    if legal > C:
        raise ValueError(f"legal length {legal} exceeds capacity {C}")
    check_standard_f(fixed_rows, off_lo, lo, hi, legal, C)
    q = q_main.reshape(B, G, h, d).contiguous()
    q_cat = q_pre.reshape(B, G, h * d).contiguous()
    k_new = None
    if k_pre_new is not None:
        if tuple(k_pre_new.shape) != (B, G, 1, d) or k_pre_new.dtype != idx_dt:
            raise ValueError(f"k_pre_new must be a {idx_dt} [B, G, 1, d] tensor")
        k_new = k_pre_new.reshape(B, G, d).contiguous()
        wc = int(write_col) if write_col >= 0 else C + int(write_col)
        if not 0 <= wc < C or lo <= wc < hi:
            raise ValueError(f"write_col={write_col} must lie in [0, C) and outside [lo, hi)")
    else:
        wc = 0
    P = hip_attend.sparse_partitions(B * G, S, h, merged=k > 0) if partitions is None else int(partitions)
    sc = float(1.0 / math.sqrt(d) if scale is None else scale)
    order = nat.ORDER_POSITION if canonical_order else nat.ORDER_SCORE
    nbytes = nat.lib().attnlab_sparse_decode_workspace(B, G, h, lo, hi, legal, k, P)
    wsp = _STEP_WS if workspace is None else workspace
    ws = wsp.bytes(k_cache.device, nbytes, "step")
    # select state: zeroed once, left zeroed by each call
    state = wsp.bytes(k_cache.device, B * G * nat.SELECT_STATE_WORDS * 4, "state")
    out = torch.empty(B, G, h, d, dtype=torch.bfloat16, device=k_cache.device)
    flat = torch.empty(B * G * S, dtype=torch.int64, device=k_cache.device) if return_rows else None
    entry = "attnlab_sparse_decode_step" if idx_dt == torch.bfloat16 else "attnlab_sparse_decode_step_f32"
    # contiguous copies (if any) are held here: a temporary's memory could go to the next one before the launch
    wq_c, wk_c = wq_t_scaled.contiguous(), wk.contiguous()
    nat.call(entry, q.data_ptr(), q_cat.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
             zT.data_ptr(), wq_c.data_ptr(), wk_c.data_ptr(), nat.ptr(k_new), B, G, h, r,
             C, lo, hi, legal, k, wc, sc, order, P, state.data_ptr(), ws.data_ptr(), ws.numel(), None, nat.ptr(flat),
             out.data_ptr(), nat.stream_of(k_cache.device))
    out = out.view(B, G, h, 1, d)
    return (out, flat) if return_rows else out


def sparse_decode_step(q_main, q_pre, k_cache, v_cache, zT, indexer: GroupedIndexer, request: DecodeRequest, *,
                       k_pre_new=None, scale=None, backend="sdpa"):
    return sparse_decode_step_kernel(q_main, q_pre, k_cache, v_cache, zT, indexer.wq_t_scaled, indexer.wk,
                                     request.fixed_rows, request.off_lo, request.layout.candidate_lo,
                                     request.layout.candidate_hi, request.k, request.selected_count,
                                     k_pre_new=k_pre_new, write_col=request.write_col, scale=scale, backend=backend)


def dense_decode_step(q_main, k_cache, v_cache, valid_length: int, *, backend="sdpa_fold", scale=None):
    """One layer's A read for one new query: every valid position, on the dense decode kernel."""
    from .full import full_attention
    return full_attention(q_main, k_cache, v_cache, valid_length=valid_length, backend=backend, scale=scale)
