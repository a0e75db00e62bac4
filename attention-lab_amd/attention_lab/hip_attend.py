"""Gather-free decode attention on gfx950: the HIP replacement of the reference's Metal P1 kernels.

`HipAttend.__call__` keeps the signature, shapes, dtypes and ValueError contract of `MetalAttend.__call__`
(src/attention_lab/metal_attend.py:177-250), including the interleaved [G, C, 2, d] diagnostic layout, and
`model_views` is the same batch-1 adapter (metal_attend.py:253-259). Limits are wider than the Metal kernel's:
h <= 8 query heads per group (Metal: 4). Listed positions outside [0, C) are skipped by the kernel, never read.

Beyond the reference: `attend` (batched [B,G,...] form) and `dense_decode` (the full read A for one decode query),
both on the same kernel.
"""
from __future__ import annotations

import math

import torch

from . import _native as nat

TG = 256          # threads per block
HEAD_DIM = 128    # 8 lanes x 16 dims
MAX_H = 8
MAX_P = 64        # partitions accepted by the MetalAttend-compatible entry point
MAX_P_DENSE = 256


def available() -> bool:
    return nat.gpu_available()


def _check_kv(KV, q, rows, partitions):
    """Interleaved layout KV [G, C, 2*d] (metal_attend.py:177-189)."""
    G, C, dd = KV.shape
    if dd != 2 * HEAD_DIM:
        raise ValueError("interleaved rows must hold K and V of head_dim 128")
    h = int(q.shape[1]) if q.dim() == 3 else -1
    if q.dim() != 3 or q.shape[0] != G or q.shape[2] != HEAD_DIM or q.dtype != torch.bfloat16 or not q.is_contiguous() \
            or not 1 <= h <= MAX_H:
        raise ValueError(f"q must be a contiguous bfloat16 [G, h, 128] tensor with h <= {MAX_H}")
    if rows.dim() != 2 or rows.shape[0] != G or rows.dtype != torch.int32 or not rows.is_contiguous() or rows.shape[1] < 1:
        raise ValueError("rows must be a contiguous int32 [G, S] tensor with S >= 1")
    if not 1 <= int(partitions) <= MAX_P:
        raise ValueError(f"partitions must be in [1, {MAX_P}]")
    return G, C, h, int(rows.shape[1])


def _check(K, V, q, rows, partitions):
    """Separate-buffer layout K, V [G, C, d] (metal_attend.py:192-215)."""
    if K.dim() != 3 or K.dtype != torch.bfloat16 or not K.is_contiguous():
        raise ValueError("K must be a contiguous bfloat16 [G, C, d] tensor (batch 1)")
    if V.shape != K.shape or V.dtype != torch.bfloat16 or not V.is_contiguous():
        raise ValueError("V must match K")
    G, C, d = K.shape
    if d != HEAD_DIM:
        raise ValueError(f"head_dim must be {HEAD_DIM} (8 lanes x 16)")
    if q.dim() != 3 or q.shape[0] != G or q.shape[2] != d or q.dtype != torch.bfloat16 or not q.is_contiguous():
        raise ValueError("q must be a contiguous bfloat16 [G, h, d] tensor")
    h = int(q.shape[1])
    if not 1 <= h <= MAX_H:
        raise ValueError(f"h must be in [1, {MAX_H}]")
    if rows.dim() != 2 or rows.shape[0] != G or rows.dtype != torch.int32 or not rows.is_contiguous():
        raise ValueError("rows must be a contiguous int32 [G, S] tensor of original positions")
    S = int(rows.shape[1])
    if S < 1:
        raise ValueError("at least one row must be selected")
    if not 1 <= int(partitions) <= MAX_P:
        raise ValueError(f"partitions must be in [1, {MAX_P}]")
    for t in (V, q, rows):
        if t.device != K.device:
            raise ValueError("all inputs must live on the same device")
    if not K.is_cuda:
        raise ValueError("inputs must live on a HIP device")
    return G, C, h, S


def _out(out, shape, dtype, device):
    if dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("out_dtype must be float32 or bfloat16")
    if out is None:
        return torch.empty(*shape, dtype=dtype, device=device)
    if tuple(out.shape) != tuple(shape) or out.dtype != dtype or not out.is_contiguous() or out.device != device:
        raise ValueError(f"out must be a contiguous {dtype} tensor of shape {tuple(shape)}")
    return out


def _part(part, n, device):
    if part is None:
        return torch.empty(max(n, 1), dtype=torch.float32, device=device)
    if part.dtype != torch.float32 or not part.is_contiguous() or part.numel() < n or part.device != device:
        raise ValueError(f"part must be a contiguous float32 tensor of at least {n} elements")
    return part


class HipAttend:
    """Gather-free subset attention: out[g, i] = softmax(q[g, i] . K[g, rows[g]] * scale) @ V[g, rows[g]]."""

    def __init__(self):
        if not available():
            raise RuntimeError("needs a HIP device and the built libattnlab.so")

    def __call__(self, K, V, q, rows, *, scale=None, partitions: int = 4, out_dtype=torch.float32, out=None, part=None,
                 kv_interleaved=None):
        """K, V [G, C, d] bf16; or `kv_interleaved` [G, C, 2, d] bf16 (K then V per position) with K and V ignored."""
        if kv_interleaved is not None:
            kv = kv_interleaved
            if kv.dim() != 4 or kv.shape[2] != 2 or kv.dtype != torch.bfloat16 or not kv.is_contiguous():
                raise ValueError("kv_interleaved must be a contiguous bfloat16 [G, C, 2, d] tensor")
            base = kv.view(kv.shape[0], kv.shape[1], 2 * kv.shape[3])
            G, C, h, S = _check_kv(base, q, rows, partitions)
            if not base.is_cuda or q.device != base.device or rows.device != base.device:
                raise ValueError("inputs must live on one HIP device")
            k_ptr, v_ptr, row_stride = base.data_ptr(), base.data_ptr() + HEAD_DIM * 2, 2 * HEAD_DIM
            device = base.device
        else:
            G, C, h, S = _check(K, V, q, rows, partitions)
            k_ptr, v_ptr, row_stride = K.data_ptr(), V.data_ptr(), HEAD_DIM
            device = K.device
        P = int(partitions)
        sc = float(1.0 / math.sqrt(HEAD_DIM) if scale is None else scale)
        out = _out(out, (G, h, HEAD_DIM), out_dtype, device)
        part = _part(part, G * P * h * (HEAD_DIM + 2) if P > 1 else 0, device)
        nat.call("attnlab_attend", k_ptr, v_ptr, C * row_stride, row_stride, q.data_ptr(), rows.data_ptr(), S, 1, G, h,
                 S, C, P, sc, out.data_ptr(), int(out.dtype == torch.bfloat16), part.data_ptr(), nat.stream_of(device))
        return out


def model_views(K4, V4, q5, rows3):
    """Model-side tensors (batch 1) -> kernel views: K/V [G, C, d], q [G, h, d], rows int32 [G, S]."""
    if K4.shape[0] != 1 or q5.shape[0] != 1 or rows3.shape[0] != 1:
        raise ValueError("the batch-1 attend op takes batch 1 (use attend for batches)")
    if q5.shape[3] != 1:
        raise ValueError("one query position per step")
    return K4[0], V4[0], q5[0, :, :, 0, :].contiguous(), rows3[0].to(torch.int32).contiguous()


# ---------------------------------------------------------------------------------------------------------------------
# batched forms
# ---------------------------------------------------------------------------------------------------------------------
def reference_attend(K, V, q, rows, *, scale=None):
    """float32 CPU check of HipAttend from the same inputs (metal_attend.py:262-273): K/V [G,C,d], q [G,h,d], rows
    [G,S] -> [G,h,d], softmax over the listed rows only, read by original position. Not a compute path."""
    Kf, Vf, qf = (t.detach().float().cpu() for t in (K, V, q))
    r = rows.detach().long().cpu()
    sc = 1.0 / math.sqrt(K.shape[-1]) if scale is None else float(scale)
    out = torch.empty(qf.shape)
    for g in range(qf.shape[0]):
        s = torch.einsum("id,sd->is", qf[g], Kf[g, r[g]]) * sc
        out[g] = torch.softmax(s, dim=-1) @ Vf[g, r[g]]
    return out


_SHARED_WS = nat.Workspace()


def _check_cache(k, v, q):
    if k.dim() != 4 or k.dtype != torch.bfloat16 or not k.is_contiguous() or not k.is_cuda:
        raise ValueError("the cache must be a contiguous bfloat16 [B, G, C, d] tensor on a HIP device")
    if v.shape != k.shape or v.dtype != k.dtype or not v.is_contiguous() or v.device != k.device:
        raise ValueError("v must match k")
    B, G, C, d = k.shape
    if d != HEAD_DIM:
        raise ValueError(f"head_dim must be {HEAD_DIM}")
    if q.dim() != 4 or tuple(q.shape[:2]) != (B, G) or q.shape[3] != d or q.dtype != torch.bfloat16 \
            or not q.is_contiguous() or q.device != k.device:
        raise ValueError("q must be a contiguous bfloat16 [B, G, h, d] tensor on the cache device")
    h = int(q.shape[2])
    if not 1 <= h <= MAX_H:
        raise ValueError(f"h must be in [1, {MAX_H}]")
    return B, G, C, h


def auto_partitions(BG: int, rows: int, *, max_p: int, min_rows: int, blocks: int = 256) -> int:
    """Split-K count: about `blocks` workgroups over the chip, each with >= min_rows rows.

    Measured on MI355X (256 CUs): the sparse read is fastest with about one workgroup per CU and >= 128 rows each
    (more partitions add per-workgroup start-up and merge cost); the dense read with about four per CU and >= 1024
    rows each. Use sparse_partitions / dense_partitions.
    """
    want = -(-blocks // max(BG, 1))
    cap = max(1, rows // min_rows)
    return max(1, min(max_p, want, cap))


def sparse_partitions(BG: int, rows: int, h: int = 1, merged: bool = False) -> int:
    """Split-K count of the sparse read. `merged`: for the fused decode step, whose attend merges its partials in-kernel
    (no combine launch) - see merged_partitions. Otherwise (the standalone attend, merged by the combine kernel): The kernel also splits each (b, g) over up to h head groups (powers of two
    dividing h) until the grid reaches one workgroup per CU; those count towards the 256 workgroups. With four head
    groups and at least 32 (b, g) rows the target is 512: splitting the rows further beats splitting the heads there
    (MI355X, 32K, S = 1092, per layer: B=4, h=4 33.2 us at P=4 against 34.1 at P=2; B=8 48.8 at P=2 against 49.5 at
    P=1; with eight head groups, B=4, the 256 target is 0.2 us better). With one head per KV group and at least 128
    (b, g) rows it is 128 (B=16, h=1: 73.7 us at P=1 against 74.3 at P=2; B=8 keeps P=4, 45.6 us)."""
    if merged:
        return merged_partitions(BG, rows, h)
    hg = h & -h if h > 0 else 1   # largest power of two dividing h
    blocks = 512 if hg == 4 and BG >= 32 else 128 if hg == 1 and BG >= 128 else 256
    return auto_partitions(BG * hg, rows, max_p=MAX_P, min_rows=128, blocks=blocks)


def merged_partitions(BG: int, rows: int, h: int = 1) -> int:
    """Split-K count of the fused step's attend (partials merged in-kernel by the last partition to arrive). About 256
    workgroups over the chip, split by rows first (each row read once) and by head groups after (the kernel adds head
    groups, which read the same rows twice, until the grid reaches 256); at least 128 rows per partition, at most 16
    partitions, or 8 with four or more heads per KV group, where two head groups also come first from 32 (b, g) rows
    on (a four-head workgroup's arithmetic then costs more than the second read).
    Measured on MI355X, step per layer, the rule's P against the best of P in {1, 2, 4, 8, 16, 32}:
    32K (S = 1092): B=1..2 P=8 best for h = 1, 2, 4; B=4 h=1 P=8 (30.8 us), h=2 P=8 31.79 against P=4 31.45, h=4
    P=4 (32.8); B=8 P=4 / 4 / 2 best for h = 1 / 2 / 4; B=16 P=2 / 2 / 1 best (h=1 70.39 against 72.14 at P=1).
    128K (S = 4164): B=1 h=2 P=16 best (40.39), h=4 P=8 40.9 against P=16 40.69; B=2 h=2 P=16 54.57 against P=8
    54.2, h=4 P=8 best (56.04; 59.58 at P=4); B=4 h=2 P=8 best (93.11), h=4 P=4 best (95.36)."""
    hg = h & -h if h > 0 else 1
    q = 2 if hg >= 4 and BG >= 32 else 1
    max_p = 8 if hg >= 4 else 16
    return auto_partitions(BG * q, rows, max_p=max_p, min_rows=128, blocks=256)


def dense_partitions(BG: int, length: int) -> int:
    return auto_partitions(BG, length, max_p=MAX_P_DENSE, min_rows=1024, blocks=1024)


def attend(q, k, v, rows, *, scale=None, partitions=None, out=None, out_dtype=torch.bfloat16, workspace=None):
    """Batched gather-free attention: q [B,G,h,d], k/v [B,G,C,d] bf16, rows int32 [B,G,S] -> out [B,G,h,d]."""
    B, G, C, h = _check_cache(k, v, q)
    if rows.dim() != 3 or tuple(rows.shape[:2]) != (B, G) or rows.dtype != torch.int32 or not rows.is_contiguous() \
            or rows.device != k.device:
        raise ValueError("rows must be a contiguous int32 [B, G, S] tensor on the cache device")
    S = int(rows.shape[2])
    if S < 1:
        raise ValueError("at least one row must be selected")
    P = sparse_partitions(B * G, S, h) if partitions is None else int(partitions)
    if not 1 <= P <= MAX_P:
        raise ValueError(f"partitions must be in [1, {MAX_P}]")
    ws = _SHARED_WS if workspace is None else workspace
    out = _out(out, (B, G, h, HEAD_DIM), out_dtype, k.device)
    part = ws.bytes(k.device, B * G * P * h * (HEAD_DIM + 2) * 4, "attend_part") if P > 1 else None
    sc = float(1.0 / math.sqrt(HEAD_DIM) if scale is None else scale)
    nat.call("attnlab_attend", k.data_ptr(), v.data_ptr(), C * HEAD_DIM, HEAD_DIM, q.data_ptr(), rows.data_ptr(), S,
             B, G, h, S, C, P, sc, out.data_ptr(), int(out.dtype == torch.bfloat16), nat.ptr(part),
             nat.stream_of(k.device))
    return out


def attend_paged(q, k_pages, v_pages, block_table, rows=None, *, length=None, scale=None, partitions=None, out=None,
                 out_dtype=torch.bfloat16, workspace=None):
    """Gather-free attention over a paged cache: q [B,G,h,d]; k_pages / v_pages [num_pages, G, page_size, d] bf16 pools;
    block_table int32 [B, max_pages] (the pool page of each sequence's logical page); rows int32 [B,G,S] positions, or
    None with `length` for the dense read of positions [0, length). -> out [B,G,h,d]. Listed positions on a page entry
    outside [0, num_pages) (e.g. -1 for unmapped) are skipped."""
    if q.dim() != 4 or q.dtype != torch.bfloat16 or not q.is_contiguous() or q.shape[3] != HEAD_DIM:
        raise ValueError("q must be a contiguous bfloat16 [B, G, h, 128] tensor")
    B, G, h, _ = q.shape
    if not 1 <= h <= MAX_H:
        raise ValueError(f"h must be in [1, {MAX_H}]")
    if (k_pages.dim() != 4 or k_pages.dtype != torch.bfloat16 or not k_pages.is_contiguous() or k_pages.shape[1] != G
            or k_pages.shape[3] != HEAD_DIM or v_pages.shape != k_pages.shape or v_pages.dtype != torch.bfloat16
            or not v_pages.is_contiguous()):
        raise ValueError("k_pages / v_pages must be contiguous bfloat16 [num_pages, G, page_size, 128] pools")
    num_pages, page = int(k_pages.shape[0]), int(k_pages.shape[2])
    if page & (page - 1):
        raise ValueError("page_size must be a power of two")
    if (block_table.dim() != 2 or block_table.shape[0] != B or block_table.dtype != torch.int32
            or block_table.stride(1) != 1):
        raise ValueError("block_table must be an int32 [B, max_pages] tensor with unit column stride")
    max_pages = int(block_table.shape[1])
    for t in (k_pages, v_pages, block_table):
        if t.device != q.device:
            raise ValueError("all inputs must live on one device")
    if rows is None:
        if length is None or not 1 <= int(length) <= max_pages * page:
            raise ValueError("without rows, length must be in [1, max_pages * page_size]")
        S, rows_ptr, rows_stride = int(length), None, 0
    else:
        if rows.dim() != 3 or tuple(rows.shape[:2]) != (B, G) or rows.dtype != torch.int32 or not rows.is_contiguous():
            raise ValueError("rows must be a contiguous int32 [B, G, S] tensor")
        S, rows_ptr, rows_stride = int(rows.shape[2]), rows.data_ptr(), int(rows.shape[2])
        if S < 1:
            raise ValueError("at least one row must be selected")
    P = sparse_partitions(B * G, S, h) if partitions is None else int(partitions)
    if not 1 <= P <= MAX_P:
        raise ValueError(f"partitions must be in [1, {MAX_P}]")
    ws = _SHARED_WS if workspace is None else workspace
    out = _out(out, (B, G, h, HEAD_DIM), out_dtype, q.device)
    part = ws.bytes(q.device, B * G * P * h * (HEAD_DIM + 2) * 4, "attend_part") if P > 1 else None
    sc = float(1.0 / math.sqrt(HEAD_DIM) if scale is None else scale)
    nat.call("attnlab_attend_paged", k_pages.data_ptr(), v_pages.data_ptr(), num_pages, page, block_table.data_ptr(),
             block_table.stride(0), max_pages, q.data_ptr(), rows_ptr, rows_stride, B, G, h, S, P, sc, out.data_ptr(),
             int(out.dtype == torch.bfloat16), nat.ptr(part), nat.stream_of(q.device))
    return out


def page_cache(k, v, page_size: int, *, spare_pages: int = 0, generator=None, fill=float("nan")):
    """Copy a contiguous cache k, v [B,G,C,d] into pools of pages [B*ceil(C/page)+spare, G, page, d] placed in a
    random order, with the block table [B, ceil(C/page)] int32 that finds them; unused pool pages hold `fill`. A
    layout helper for tests and benches (one copy of the cache)."""
    B, G, C, d = k.shape
    npg = -(-C // page_size)
    num = B * npg + int(spare_pages)
    perm = torch.randperm(num, generator=generator)[:B * npg].view(B, npg).to(torch.int32)
    kp = torch.full((num, G, page_size, d), fill, dtype=k.dtype, device=k.device)
    vp = torch.full_like(kp, fill)
    pad = npg * page_size - C
    kk = torch.nn.functional.pad(k, (0, 0, 0, pad)) if pad else k
    vv = torch.nn.functional.pad(v, (0, 0, 0, pad)) if pad else v
    idx = perm.to(k.device).long()
    kp[idx.reshape(-1)] = kk.view(B, G, npg, page_size, d).permute(0, 2, 1, 3, 4).reshape(B * npg, G, page_size, d)
    vp[idx.reshape(-1)] = vv.view(B, G, npg, page_size, d).permute(0, 2, 1, 3, 4).reshape(B * npg, G, page_size, d)
    return kp, vp, perm.to(k.device)


def dense_decode(q, k, v, valid_length: int, *, scale=None, partitions=None, out=None, out_dtype=torch.bfloat16,
                 workspace=None):
    """Dense decode read A over positions [0, valid_length): q [B,G,h,d], k/v [B,G,C,d] -> out [B,G,h,d]."""
    B, G, C, h = _check_cache(k, v, q)
    L = int(valid_length)
    if not 0 < L <= C:
        raise ValueError(f"valid_length={L} must be in (0, capacity={C}]")
    P = dense_partitions(B * G, L) if partitions is None else int(partitions)
    if not 1 <= P <= MAX_P_DENSE:
        raise ValueError(f"partitions must be in [1, {MAX_P_DENSE}]")
    ws = _SHARED_WS if workspace is None else workspace
    out = _out(out, (B, G, h, HEAD_DIM), out_dtype, k.device)
    part = ws.bytes(k.device, B * G * P * h * (HEAD_DIM + 2) * 4, "dense_part") if P > 1 else None
    sc = float(1.0 / math.sqrt(HEAD_DIM) if scale is None else scale)
    nat.call("attnlab_dense_decode", k.data_ptr(), v.data_ptr(), C * HEAD_DIM, HEAD_DIM, q.data_ptr(), B, G, h, L, C,
             P, sc, out.data_ptr(), int(out.dtype == torch.bfloat16), nat.ptr(part), nat.stream_of(k.device))
    return out


PREFILL_HEADS = (1, 2, 4, 8, 16)


PREFILL_ROWS = 128          # (query, head) rows per workgroup of the prefill kernel
PREFILL_MAX_SPLITS = 16


def prefill_splits(B: int, G: int, h: int, T: int, q_pos0: int, valid_length: int) -> int:
    """Key splits of the causal prefill read: none once the query tiles give a workgroup per CU (256); below that as
    many as bring the grid to about two workgroups per CU, each split at least 512 keys of the longest tile's visible
    range. A 1K chunk after 7K cached positions at B=1, G=8, h=2 (128 tiles) takes 4."""
    tiles = B * G * -(-T // (PREFILL_ROWS // h))
    if tiles >= 256:
        return 1
    keys = min(valid_length, q_pos0 + T)
    s = min(PREFILL_MAX_SPLITS, 512 // max(tiles, 1), keys // 512)
    return s if s >= 2 else 1


def prefill_attend(q, k, v, q_pos0: int, valid_length: int, *, scale=None, out=None, splits=None, workspace=None):
    """Causal prefill read on the matrix cores: q [B,G,h,T,d] at positions q_pos0 .. q_pos0 + T - 1, k/v [B,G,C,d];
    query t reads the cache rows j <= q_pos0 + t, j < valid_length. Returns bf16 [B,G,h,T,d]. A grid too small to fill
    the chip splits each tile's keys (prefill_splits; `splits` overrides it) and merges the splits' partials, held in
    the workspace, in a second kernel."""
    if k.dim() != 4 or k.dtype != torch.bfloat16 or not k.is_contiguous() or not k.is_cuda:
        raise ValueError("the cache must be a contiguous bfloat16 [B, G, C, d] tensor on a HIP device")
    if v.shape != k.shape or v.dtype != k.dtype or not v.is_contiguous() or v.device != k.device:
        raise ValueError("v must match k")
    B, G, C, d = k.shape
    if d != HEAD_DIM:
        raise ValueError(f"head_dim must be {HEAD_DIM}")
    if q.dim() != 5 or tuple(q.shape[:2]) != (B, G) or q.shape[4] != d or q.dtype != torch.bfloat16 \
            or not q.is_contiguous() or q.device != k.device:
        raise ValueError("q must be a contiguous bfloat16 [B, G, h, T, d] tensor on the cache device")
    h, T = int(q.shape[2]), int(q.shape[3])
    if h not in PREFILL_HEADS:
        raise ValueError(f"h={h} must be one of {PREFILL_HEADS}")
    L, p0 = int(valid_length), int(q_pos0)
    if not 0 < L <= C or p0 < 0:
        raise ValueError(f"need 0 < valid_length <= capacity and q_pos0 >= 0 (got {L}, {C}, {p0})")
    if out is None:
        out = torch.empty(B, G, h, T, d, dtype=torch.bfloat16, device=k.device)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != tuple(q.shape) or not out.is_contiguous():
        raise ValueError("out must be a contiguous bfloat16 tensor shaped like q")
    sc = float(1.0 / math.sqrt(HEAD_DIM) if scale is None else scale)
    ns = prefill_splits(B, G, h, T, p0, L) if splits is None else int(splits)
    if not 1 <= ns <= PREFILL_MAX_SPLITS:
        raise ValueError(f"splits must be in [1, {PREFILL_MAX_SPLITS}]")
    if ns == 1:
        nat.call("attnlab_prefill_attend", q.data_ptr(), k.data_ptr(), v.data_ptr(), C * d, d, out.data_ptr(), B, G, h,
                 T, d, p0, L, C, sc, nat.stream_of(k.device))
        return out
    nbytes = nat.lib().attnlab_prefill_part_bytes(B, G, h, T, ns)
    ws = _SHARED_WS if workspace is None else workspace
    part = ws.bytes(k.device, nbytes, "prefill_part")
    nat.call("attnlab_prefill_attend_split", q.data_ptr(), k.data_ptr(), v.data_ptr(), C * d, d, out.data_ptr(), B, G,
             h, T, d, p0, L, C, sc, ns, part.data_ptr(), int(part.numel()), nat.stream_of(k.device))
    return out
