"""Index score ops on gfx950: the HIP replacement of the reference's Metal P0 kernels.

`HipScore.fused` / `HipScore.two_launch` keep the signatures, shapes, dtypes and ValueError contract of
`MetalScore.fused` / `MetalScore.two_launch` (src/attention_lab/metal_score.py:254-330), and `model_views` is the
same batch-1 adapter (metal_score.py:333-341). One difference is deliberate: the reference's `fused` returns without
launching when the candidate range is empty (metal_score.py:304-305) and so never writes the z column in that case,
while `two_launch` does write it; both HIP entry points write the z column whenever they are called, which is what
the PyTorch path (decode.py:156-157) does.

Beyond the reference: `score_grouped` is the batched form ([B,G,r,C] tables, used by the decode step) and
`score_lightning` the DeepSeek-style lightning indexer (ReLU, per-head weights, fp16/bf16 keys), for which the
reference has no kernel.
"""
from __future__ import annotations

import math

import torch

from . import _native as nat

TG = 256     # threads per block of the scan kernel
MAX_R = 32   # widest index the kernels take


def available() -> bool:
    return nat.gpu_available()


def _on_device(t, like, name):
    if not t.is_cuda or t.device != like.device:
        raise ValueError(f"{name} must live on the same HIP device as zT")


def _check(zT, k_new, wk, q_cat, wq_t, lo, hi, write_col):
    """Batch-1 contract of MetalScore (metal_score.py:254-271), plus the device check of a HIP op."""
    if zT.dim() != 3 or zT.dtype != torch.bfloat16 or not zT.is_contiguous():
        raise ValueError("zT must be a contiguous bfloat16 [G, r, C] tensor (batch 1)")
    G, r, C = zT.shape
    if r > MAX_R:
        raise ValueError(f"index width {r} exceeds the kernel's {MAX_R}")
    if tuple(k_new.shape) != (G, wk.shape[2]) or tuple(wk.shape[:2]) != (G, r):
        raise ValueError("k_new must be [G, d] and wk [G, r, d]")
    if q_cat.dim() != 2 or q_cat.shape[0] != G or tuple(wq_t.shape) != (G, q_cat.shape[1], r):
        raise ValueError("q_cat must be [G, hd] and wq_t [G, hd, r]")
    for t in (k_new, wk, q_cat, wq_t):
        if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.device != zT.device:
            raise ValueError("every input must be contiguous bfloat16 on the same device as zT")
    if not zT.is_cuda:
        raise ValueError("zT must live on a HIP device")
    if not (0 <= lo <= hi <= C and 0 <= write_col < C):
        raise ValueError(f"need 0 <= lo <= hi <= C and 0 <= write_col < C, got lo={lo} hi={hi} write_col={write_col} C={C}")
    if lo <= write_col < hi:
        raise ValueError("write_col must lie outside the scanned range [lo, hi)")
    return G, r, C, int(wk.shape[2]), int(q_cat.shape[1])


def _out_buffer(out, rows, M, device):
    if out is None:
        return torch.empty(rows, max(M, 1), dtype=torch.float32, device=device)
    if out.dtype != torch.float32 or out.device != device or out.dim() != 2 or out.shape[0] != rows \
            or out.shape[1] < M or out.stride(1) != 1:
        raise ValueError(f"out must be a float32 [{rows}, >= {M}] tensor with unit column stride on the zT device")
    return out


class HipScore:
    """Scoring segment of the D chain: `fused` is one launch, `two_launch` is prologue + scan."""

    def __init__(self):
        if not available():
            raise RuntimeError("needs a HIP device and the built libattnlab.so")

    @staticmethod
    def vector_ok(C: int, lo: int) -> bool:
        """The 16-byte-load scan needs 16-byte aligned table rows (C % 8 == 0); lo may be anything."""
        return C % 8 == 0

    def fused(self, zT, k_new, wk, q_cat, wq_t, lo: int, hi: int, write_col: int, out=None, version: int = 2):
        """Write z of the newest key into zT[:, :, write_col] and return fp32 scores [G, hi - lo] of the candidates.

        version 2: 16-byte loads (falls back to 2-byte loads when C % 8 != 0); version 1: 2-byte loads.
        """
        G, r, C, d, hd = _check(zT, k_new, wk, q_cat, wq_t, lo, hi, write_col)
        M = hi - lo
        out = _out_buffer(out, G, M, zT.device)
        nat.call("attnlab_score_grouped", zT.data_ptr(), k_new.data_ptr(), wk.data_ptr(), q_cat.data_ptr(),
                 wq_t.data_ptr(), None, None, out.data_ptr(), out.stride(0), 1, G, r, C, d, hd, lo, hi, write_col,
                 int(version == 2), None, nat.stream_of(zT.device))
        return out[:, :M]

    def two_launch(self, zT, k_new, wk, q_cat, wq_t, lo: int, hi: int, write_col: int, out=None, u_buf=None,
                   version: int = 2):
        G, r, C, d, hd = _check(zT, k_new, wk, q_cat, wq_t, lo, hi, write_col)
        M = hi - lo
        if u_buf is None:
            u_buf = torch.empty(G, r, dtype=torch.float32, device=zT.device)
        elif u_buf.dtype != torch.float32 or tuple(u_buf.shape) != (G, r) or not u_buf.is_contiguous() \
                or u_buf.device != zT.device:
            raise ValueError(f"u_buf must be a contiguous float32 [{G}, {r}] tensor on the zT device")
        out = _out_buffer(out, G, M, zT.device)
        s = nat.stream_of(zT.device)
        nat.call("attnlab_score_prologue", zT.data_ptr(), k_new.data_ptr(), wk.data_ptr(), q_cat.data_ptr(),
                 wq_t.data_ptr(), u_buf.data_ptr(), 1, G, r, C, d, hd, write_col, s)
        if M > 0:
            nat.call("attnlab_score_grouped", zT.data_ptr(), None, wk.data_ptr(), None, None, u_buf.data_ptr(), None,
                     out.data_ptr(), out.stride(0), 1, G, r, C, d, hd, lo, hi, write_col, int(version == 2), None, s)
        return out[:, :M]


def model_views(zT4, k_pre_new4, q_pre5, indexer):
    """Model-side tensors (batch 1) -> the kernel's views, as metal_score.model_views (metal_score.py:333-341)."""
    if zT4.shape[0] != 1:
        raise ValueError("the batch-1 score op takes batch 1 (use score_grouped for batches)")
    zT = zT4[0]
    k_new = k_pre_new4[0, :, 0, :]
    B, G, h, T, d = q_pre5.shape
    q_cat = q_pre5[0].permute(0, 2, 1, 3).reshape(G, T * h * d)
    return zT, k_new.contiguous(), indexer.wk, q_cat.contiguous(), indexer.wq_t_scaled


# ---------------------------------------------------------------------------------------------------------------------
# batched ops
# ---------------------------------------------------------------------------------------------------------------------
def _check_batched(zT, wk, q_cat, wq_t, k_new, u):
    """Shapes of the batched score. The index table and its inputs are all bfloat16 (the reference's random indexers)
    or all float32 (a trained bank's table, trained.py:78-81)."""
    if zT.dim() != 4 or zT.dtype not in (torch.bfloat16, torch.float32) or not zT.is_contiguous() or not zT.is_cuda:
        raise ValueError("zT must be a contiguous bfloat16 or float32 [B, G, r, C] tensor on a HIP device")
    dt = zT.dtype
    name = "bfloat16" if dt == torch.bfloat16 else "float32"
    B, G, r, C = zT.shape
    if r > MAX_R:
        raise ValueError(f"index width {r} exceeds the kernel's {MAX_R}")
    d = 0
    if k_new is not None:
        if wk is None or wk.dtype != dt or not wk.is_contiguous() or wk.dim() != 3 or tuple(wk.shape[:2]) != (G, r):
            raise ValueError(f"writing the z column needs wk, a contiguous {name} [G, r, d] tensor")
        d = int(wk.shape[2])
        if tuple(k_new.shape) != (B, G, d) or k_new.dtype != dt or not k_new.is_contiguous():
            raise ValueError(f"k_new must be a contiguous {name} [B, G, d] tensor")
        _on_device(k_new, zT, "k_new")
        _on_device(wk, zT, "wk")
    if u is None:
        if q_cat is None or q_cat.dim() != 3 or tuple(q_cat.shape[:2]) != (B, G) or q_cat.dtype != dt \
                or not q_cat.is_contiguous():
            raise ValueError(f"q_cat must be a contiguous {name} [B, G, hd] tensor")
        hd = int(q_cat.shape[2])
        if wq_t is None or tuple(wq_t.shape) != (G, hd, r) or wq_t.dtype != dt or not wq_t.is_contiguous():
            raise ValueError(f"wq_t must be a contiguous {name} [G, hd, r] tensor")
        for t, n in ((q_cat, "q_cat"), (wq_t, "wq_t")):
            _on_device(t, zT, n)
    else:
        if u.dtype != torch.float32 or tuple(u.shape) != (B, G, r) or not u.is_contiguous():
            raise ValueError("u must be a contiguous float32 [B, G, r] tensor")
        _on_device(u, zT, "u")
        hd = 0
    return B, G, r, C, d, hd


def score_grouped(zT, lo: int, hi: int, *, wk=None, q_cat=None, wq_t=None, u=None, k_new=None, write_col: int = -1,
                  out=None, u_out=None, state=None):
    """Batched parity-mode score: optional z-column write of k_new, u from (q_cat, wq_t) or given, scan of [lo, hi).

    zT [B,G,r,C] bf16, or float32 for a trained bank (then q_cat, wq_t, wk and k_new are float32 too); q_cat [B,G,hd];
    wq_t [G,hd,r]; u [B,G,r] fp32; k_new [B,G,d]. Returns fp32 [B, G, hi-lo].
    state: optional zeroed int32 select state [B, G, SELECT_STATE_WORDS] that receives the scores' first-digit
    histogram for select_rows.
    """
    B, G, r, C, d, hd = _check_batched(zT, wk, q_cat, wq_t, k_new, u)
    lo, hi = int(lo), int(hi)
    if not 0 <= lo <= hi <= C:
        raise ValueError(f"need 0 <= lo <= hi <= C, got lo={lo} hi={hi} C={C}")
    if k_new is not None and (not 0 <= write_col < C or lo <= write_col < hi):
        raise ValueError(f"write_col={write_col} must lie in [0, C) and outside [lo, hi)")
    M = hi - lo
    if out is None:
        out = torch.empty(B, G, max(M, 1), dtype=torch.float32, device=zT.device)
    elif out.dtype != torch.float32 or out.dim() != 3 or tuple(out.shape[:2]) != (B, G) or out.shape[2] < M \
            or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous float32 [{B}, {G}, >= {M}] tensor")
    if u_out is not None and (u_out.dtype != torch.float32 or tuple(u_out.shape) != (B, G, r) or not u_out.is_contiguous()):
        raise ValueError("u_out must be a contiguous float32 [B, G, r] tensor")
    check_state(state, B, G, zT.device)
    if zT.dtype == torch.float32:
        if u is None and u_out is None and M > 0:
            u_out = torch.empty(B, G, r, dtype=torch.float32, device=zT.device)
        nat.call("attnlab_score_grouped_f32", zT.data_ptr(), nat.ptr(k_new), nat.ptr(wk), nat.ptr(q_cat),
                 nat.ptr(wq_t), nat.ptr(u), nat.ptr(u_out), out.data_ptr(), out.shape[2], B, G, r, C, d, hd, lo, hi,
                 write_col if k_new is not None else 0, nat.ptr(state), nat.stream_of(zT.device))
        return out[..., :M]
    nat.call("attnlab_score_grouped", zT.data_ptr(), nat.ptr(k_new), nat.ptr(wk), nat.ptr(q_cat), nat.ptr(wq_t),
             nat.ptr(u), nat.ptr(u_out), out.data_ptr(), out.shape[2], B, G, r, C, d, hd, lo, hi,
             write_col if k_new is not None else 0, 1, nat.ptr(state), nat.stream_of(zT.device))
    return out[..., :M]


def check_state(state, B, G, device):
    W = nat.SELECT_STATE_WORDS
    if state is not None and (state.dtype != torch.int32 or tuple(state.shape) != (B, G, W)
                              or not state.is_contiguous() or state.device != device):
        raise ValueError(f"state must be a contiguous int32 [{B}, {G}, {W}] tensor on the scores' device")


def project_queries(q_pre, wq_t_scaled):
    """u [B,G,1,r] fp32 = concat_h(q_pre) . wq_t_scaled for one decode query (indexer.py:20-24, T == 1) on the GPU."""
    B, G, h, T, d = q_pre.shape
    if T != 1:
        raise ValueError("the HIP projection takes one query position")
    dt = q_pre.dtype
    if dt not in (torch.bfloat16, torch.float32) or wq_t_scaled.dtype != dt:
        raise ValueError("q_pre and wq_t_scaled must both be bfloat16, or both float32 (a trained bank)")
    if not q_pre.is_cuda or wq_t_scaled.device != q_pre.device:
        raise ValueError("q_pre and wq_t_scaled must live on one HIP device")
    r = int(wq_t_scaled.shape[2])
    if r > MAX_R or tuple(wq_t_scaled.shape) != (G, h * d, r):
        raise ValueError(f"wq_t_scaled must be [G, h*d, r <= {MAX_R}]")
    q_cat = q_pre.reshape(B, G, h * d).contiguous()
    u = torch.empty(B, G, r, dtype=torch.float32, device=q_pre.device)
    wq = wq_t_scaled.contiguous()
    if dt == torch.float32:   # the fp32 score entry with no table and no candidates is the projection alone
        nat.call("attnlab_score_grouped_f32", None, None, None, q_cat.data_ptr(), wq.data_ptr(), None, u.data_ptr(),
                 None, 0, B, G, r, 0, d, h * d, 0, 0, 0, None, nat.stream_of(q_pre.device))
    else:
        nat.call("attnlab_score_prologue", None, None, None, q_cat.data_ptr(), wq.data_ptr(), u.data_ptr(), B, G, r,
                 0, d, h * d, 0, nat.stream_of(q_pre.device))
    return u.view(B, G, 1, r)


def candidate_scores(u, zT, lo: int, hi: int):
    """u [B,G,1,r] against the candidate columns only -> fp32 [B,G,1,hi-lo] (indexer.py:27-29) on the GPU."""
    B, G, T, r = u.shape
    if T != 1:
        raise ValueError("the HIP scan takes one query position")
    uu = u.reshape(B, G, r).float().contiguous()
    s = score_grouped(zT, lo, hi, u=uu)
    return s.view(B, G, 1, hi - lo)


def score_lightning(keys, q, w, lo: int = 0, hi=None, *, relu: bool = True, out=None):
    """Lightning-indexer score out[b,kg,t] = sum_i w[b,kg,i] * act(q[b,kg,i] . keys[b,kg,t]) for t in [lo, hi).

    keys [B,KG,L,32] fp16 or bf16 contiguous (one r-vector per position); q [B,KG,nh,32] fp32; w [B,KG,nh] fp32;
    act = ReLU when relu else identity. Returns fp32 [B, KG, hi-lo].
    """
    if keys.dim() != 4 or keys.shape[3] != 32 or keys.dtype not in (torch.float16, torch.bfloat16) \
            or not keys.is_contiguous() or not keys.is_cuda:
        raise ValueError("keys must be a contiguous fp16/bf16 [B, KG, L, 32] tensor on a HIP device")
    B, KG, L, r = keys.shape
    if q.dim() != 4 or tuple(q.shape[:2]) != (B, KG) or q.shape[3] != r or q.dtype != torch.float32 or not q.is_contiguous():
        raise ValueError("q must be a contiguous float32 [B, KG, nh, 32] tensor")
    nh = int(q.shape[2])
    if not 1 <= nh <= 8:
        raise ValueError(f"index heads nh={nh} outside [1, 8]")
    if tuple(w.shape) != (B, KG, nh) or w.dtype != torch.float32 or not w.is_contiguous():
        raise ValueError("w must be a contiguous float32 [B, KG, nh] tensor")
    for t, n in ((q, "q"), (w, "w")):
        _on_device(t, keys, n)
    hi = L if hi is None else int(hi)
    if not 0 <= lo <= hi <= L:
        raise ValueError(f"need 0 <= lo <= hi <= L, got lo={lo} hi={hi} L={L}")
    M = hi - lo
    if out is None:
        out = torch.empty(B, KG, max(M, 1), dtype=torch.float32, device=keys.device)
    dt = nat.DT_F16 if keys.dtype == torch.float16 else nat.DT_BF16
    nat.call("attnlab_score_lightning", keys.data_ptr(), dt, q.data_ptr(), w.data_ptr(), out.data_ptr(), out.shape[2],
             B, KG, L, r, nh, lo, hi, int(bool(relu)), nat.stream_of(keys.device))
    return out[..., :M]


def score_lightning_batched(keys, q, w, lo: int = 0, hi=None, *, q_pos0=None, relu: bool = True, out=None):
    """Batched (prefill) lightning score on the matrix cores, T queries per (b, kg):
    out[b,kg,t,m-lo] = sum_i w[b,kg,t,i] * act(q[b,kg,t,i] . keys[b,kg,m]) for m in [lo, hi).

    keys [B,KG,L,32] fp16 or bf16 contiguous; q [B,KG,T,nh,32] fp32 contiguous; w [B,KG,T,nh] fp32; nh in {1,2,4,8}.
    q_pos0: when given, query t sits at position q_pos0 + t and reads only keys m <= q_pos0 + t; the scores past that
    bound are not written (they keep whatever `out` held). out: optional fp32 [B,KG,T,>=hi-lo] contiguous tensor whose
    last dimension is a multiple of 4. Returns the fp32 [B, KG, T, hi-lo] view.
    """
    if keys.dim() != 4 or keys.shape[3] != 32 or keys.dtype not in (torch.float16, torch.bfloat16) \
            or not keys.is_contiguous() or not keys.is_cuda:
        raise ValueError("keys must be a contiguous fp16/bf16 [B, KG, L, 32] tensor on a HIP device")
    B, KG, L, r = keys.shape
    if q.dim() != 5 or tuple(q.shape[:2]) != (B, KG) or q.shape[4] != r or q.dtype != torch.float32 \
            or not q.is_contiguous():
        raise ValueError("q must be a contiguous float32 [B, KG, T, nh, 32] tensor")
    T, nh = int(q.shape[2]), int(q.shape[3])
    if nh not in (1, 2, 4, 8):
        raise ValueError(f"index heads nh={nh} must be 1, 2, 4 or 8")
    if tuple(w.shape) != (B, KG, T, nh) or w.dtype != torch.float32 or not w.is_contiguous():
        raise ValueError("w must be a contiguous float32 [B, KG, T, nh] tensor")
    for t, n in ((q, "q"), (w, "w")):
        _on_device(t, keys, n)
    hi = L if hi is None else int(hi)
    lo = int(lo)
    if not 0 <= lo <= hi <= L:
        raise ValueError(f"need 0 <= lo <= hi <= L, got lo={lo} hi={hi} L={L}")
    if q_pos0 is not None and int(q_pos0) < 0:
        raise ValueError(f"q_pos0={q_pos0} must be >= 0")
    M = hi - lo
    if out is None:
        out = torch.empty(B, KG, T, max((M + 3) // 4 * 4, 4), dtype=torch.float32, device=keys.device)
    elif out.dtype != torch.float32 or out.dim() != 4 or tuple(out.shape[:3]) != (B, KG, T) or out.shape[3] < M \
            or out.shape[3] % 4 or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous float32 [{B}, {KG}, {T}, >= {M}] tensor with a last dimension "
                         "that is a multiple of 4")
    else:
        _on_device(out, keys, "out")
    dt = nat.DT_F16 if keys.dtype == torch.float16 else nat.DT_BF16
    nat.call("attnlab_score_lightning_batched", keys.data_ptr(), dt, q.data_ptr(), w.data_ptr(), out.data_ptr(),
             out.shape[3], B, KG, L, r, nh, T, lo, hi, -1 if q_pos0 is None else int(q_pos0), int(bool(relu)),
             nat.stream_of(keys.device))
    return out[..., :M]


def reference_scores(zT, k_new, wk, q_cat, wq_t, lo: int, hi: int):
    """float32 CPU check of HipScore.fused from the same inputs (metal_score.py:344-350): (u [G,r], z_new [G,r],
    scores [G, hi-lo]). Not a compute path: the kernels above never call it."""
    zf, kf, wkf, qf, wqf = (t.detach().float().cpu() for t in (zT, k_new, wk, q_cat, wq_t))
    u = torch.einsum("gf,gfr->gr", qf, wqf)
    z_new = torch.einsum("grd,gd->gr", wkf, kf)
    return u, z_new, torch.einsum("gr,grm->gm", u, zf[:, :, int(lo):int(hi)])


def scale_for(r: int) -> float:
    """The 1/sqrt(r) the reference folds into wq_t_scaled (indexer.py:45)."""
    return 1.0 / math.sqrt(r)
