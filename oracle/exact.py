"""float64 numpy restatements of the hot path. Test infrastructure only.

Shapes use the reference's conventions (B batch, G KV groups, h heads per group, C capacity, d head dim, r index
width). Inputs are float arrays already holding the bf16/fp16-rounded values the device sees.
"""
from __future__ import annotations

import math

import numpy as np

from . import bf16, rules


# ---------------------------------------------------------------------------------------------------------------------
# score (parity mode)
# ---------------------------------------------------------------------------------------------------------------------
def grouped_u(q_cat: np.ndarray, wq_t: np.ndarray) -> np.ndarray:
    """u[..., g, j] = sum_f q_cat[..., g, f] * wq_t[g, f, j] (indexer.py:20-24; metal_score.py:347)."""
    return np.einsum("...gf,gfj->...gj", q_cat, wq_t)


def z_column(k_new: np.ndarray, wk: np.ndarray):
    """z[..., g, j] = sum_e wk[g, j, e] * k_new[..., g, e] (indexer.py:15-17 for one key; metal_score.py:84-89).

    Returns (float64 value, its bf16 RNE pattern as the kernel stores it).
    """
    z = np.einsum("gjd,...gd->...gj", wk, k_new)
    return z, bf16.from_f32(z.astype(np.float32))


def grouped_scores(u: np.ndarray, zT: np.ndarray, lo: int, hi: int) -> np.ndarray:
    """scores[..., g, m] = sum_j u[..., g, j] * zT[..., g, j, lo + m] (indexer.py:27-29; metal_score.py:349)."""
    return np.einsum("...gj,...gjm->...gm", u, zT[..., lo:hi])


def project_keys(k_pre: np.ndarray, wk: np.ndarray) -> np.ndarray:
    """zT [B,G,r,T] = wk . k_pre^T (indexer.py:15-17), float64."""
    return np.einsum("gjd,bgtd->bgjt", wk, k_pre)


def lightning_scores(keys: np.ndarray, q: np.ndarray, w: np.ndarray, lo: int, hi: int, relu: bool = True):
    """s[b,kg,t] = sum_i w[b,kg,i] * act(q[b,kg,i] . keys[b,kg,t]) for t in [lo, hi).

    The north_star lightning indexer; with nh = 1, w = 1 and act = identity it is grouped_scores with the key table
    transposed (the reduction the tests use to pin it).
    """
    dots = np.einsum("bkir,bktr->bkit", q, keys[:, :, lo:hi])
    if relu:
        dots = np.maximum(dots, 0.0)
    return np.einsum("bki,bkit->bkt", w, dots)


def lightning_scores_batched(keys: np.ndarray, q: np.ndarray, w: np.ndarray, lo: int, hi: int, q_pos0=None,
                             relu: bool = True) -> np.ndarray:
    """T queries per (b, kg): s[b,kg,t,m-lo] = lightning_scores of query t (q [B,KG,T,nh,r], w [B,KG,T,nh]) for m in
    [lo, hi); with q_pos0, query t sits at position q_pos0 + t and the entries m > q_pos0 + t are NaN (not scored).

    The prefill form of the north_star lightning indexer (no reference code); one query is lightning_scores.
    """
    dots = np.einsum("bktir,bkmr->bktim", q, keys[:, :, lo:hi])
    if relu:
        dots = np.maximum(dots, 0.0)
    s = np.einsum("bkti,bktim->bktm", w, dots)
    if q_pos0 is not None:
        T, M = s.shape[2], s.shape[3]
        m = lo + np.arange(M)[None, :]
        t = np.arange(T)[:, None]
        s = np.where(m <= q_pos0 + t, s, np.nan)
    return s


# ---------------------------------------------------------------------------------------------------------------------
# top-k with a defined tie order (decode.py:86-93 made deterministic)
# ---------------------------------------------------------------------------------------------------------------------
def rank_keys(scores: np.ndarray) -> np.ndarray:
    """float32 scores -> float64 ranking values: -0.0 equals +0.0, NaN ranks below -inf."""
    s = np.asarray(scores, dtype=np.float64) + 0.0  # -0.0 + 0.0 == +0.0
    return np.where(np.isnan(s), -np.inf, s), np.isnan(s)


def topk(scores: np.ndarray, k: int, order: str = "score") -> np.ndarray:
    """Indices of the k largest along the last axis; ties -> lower index; NaN below everything.

    order="score": descending score then ascending index; order="position": ascending index.
    """
    s, nan = rank_keys(scores)
    lead = s.shape[:-1]
    M = s.shape[-1]
    s2, n2 = s.reshape(-1, M), nan.reshape(-1, M)
    out = np.empty((s2.shape[0], k), dtype=np.int64)
    idx = np.arange(M)
    for i in range(s2.shape[0]):
        # primary: not-NaN first; secondary: score descending; tertiary: index ascending
        perm = np.lexsort((idx, -s2[i], n2[i]))
        sel = perm[:k]
        out[i] = np.sort(sel) if order == "position" else sel
    return out.reshape(*lead, k)


def select_rows(scores: np.ndarray, lo: int, hi: int, legal: int, k: int, order: str = "score") -> np.ndarray:
    """Row list [..., S] of original positions (decode.py:50-56, 86-93, 160-161).

    order="score": F ascending, then lo + top-k by descending score; order="position": the whole list ascending.
    """
    lead = scores.shape[:-1]
    fixed = np.array(list(range(lo)) + list(range(hi, legal)), dtype=np.int64)
    top = topk(scores, k, order="score") + lo if k > 0 else np.zeros(lead + (0,), dtype=np.int64)
    rows = np.concatenate([np.broadcast_to(fixed, lead + fixed.shape), top], axis=-1)
    if order == "position":
        rows = np.sort(rows, axis=-1)
    return rows


# ---------------------------------------------------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------------------------------------------------
def _softmax_rows(s: np.ndarray) -> np.ndarray:
    m = np.max(s, axis=-1, keepdims=True)
    e = np.exp(s - m)
    return e / np.sum(e, axis=-1, keepdims=True)


def subset_attention(q: np.ndarray, K: np.ndarray, V: np.ndarray, rows: np.ndarray, scale=None) -> np.ndarray:
    """out[b,g,i] = softmax(scale * q[b,g,i] . K[b,g,rows]) @ V[b,g,rows] (metal_attend.py:262-273).

    q [B,G,h,d], K/V [B,G,C,d], rows [B,G,S] positions; negative positions are padding and skipped.
    """
    B, G, h, d = q.shape
    sc = 1.0 / math.sqrt(d) if scale is None else float(scale)
    out = np.empty((B, G, h, d))
    for b in range(B):
        for g in range(G):
            r = rows[b, g]
            r = r[r >= 0]
            s = (q[b, g] @ K[b, g, r].T) * sc
            out[b, g] = _softmax_rows(s) @ V[b, g, r]
    return out


def dense_mask_attention(q, K, V, rows, valid_length=None, scale=None):
    """The subset read written as dense scores over [0, L) plus a -inf mask (reference.py:80-97). [B,G,h,d] out."""
    B, G, h, d = q.shape
    L = K.shape[2] if valid_length is None else int(valid_length)
    sc = 1.0 / math.sqrt(d) if scale is None else float(scale)
    keep = np.zeros((B, G, L), dtype=bool)
    for b in range(B):
        for g in range(G):
            keep[b, g, rows[b, g][rows[b, g] >= 0]] = True
    s = np.einsum("bgid,bgcd->bgic", q, K[:, :, :L]) * sc
    s = np.where(keep[:, :, None, :], s, -np.inf)
    return np.einsum("bgic,bgcd->bgid", _softmax_rows(s), V[:, :, :L])


def dense_attention(q, K, V, valid_length: int, scale=None) -> np.ndarray:
    """Full read A for one query at the last legal position (reference.py:51-62 with T == 1; full.py:17-34)."""
    B, G, h, d = q.shape
    sc = 1.0 / math.sqrt(d) if scale is None else float(scale)
    s = np.einsum("bgid,bgcd->bgic", q, K[:, :, :valid_length]) * sc
    return np.einsum("bgic,bgcd->bgid", _softmax_rows(s), V[:, :, :valid_length])


def causal_attention(q, K, V, valid_length: int, query_positions=None, scale=None) -> np.ndarray:
    """Full read A for T queries (a prefill chunk), reference.py:28-62: key j is legal for query t iff
    j <= query_positions[t] and j < valid_length; by default the queries are the last T legal positions.
    q [B,G,h,T,d] -> [B,G,h,T,d]. Written with an additive -inf mask over [0, valid_length)."""
    B, G, h, T, d = q.shape
    qp = np.arange(valid_length - T, valid_length) if query_positions is None else np.asarray(query_positions)
    sc = 1.0 / math.sqrt(d) if scale is None else float(scale)
    s = np.einsum("bgitd,bgcd->bgitc", q, K[:, :, :valid_length]) * sc
    legal = np.arange(valid_length)[None, :] <= qp[:, None]            # [T, L]
    s = np.where(legal[None, None, None], s, -np.inf)
    return np.einsum("bgitc,bgcd->bgitd", _softmax_rows(s), V[:, :, :valid_length])


# ---------------------------------------------------------------------------------------------------------------------
# whole D step (decode.py:145-163)
# ---------------------------------------------------------------------------------------------------------------------
def sparse_step(q_main, q_cat, K, V, zT, wq_t, wk, k_new, legal: int, k0: int, scale=None, order="score"):
    """One layer's D read: z column, u, scores, top-k, row list, subset attention.

    Returns dict(z_bits, scores (float64), rows, out). zT is not modified; the z column is computed for the caller
    to compare. The scan never reads write_col = legal - 1 (it lies in F).
    """
    lo, hi, k, S = rules.step(legal, k0)
    z, z_bits = z_column(k_new, wk)
    u = grouped_u(q_cat, wq_t)
    scores = grouped_scores(u, zT, lo, hi)
    rows = select_rows(scores.astype(np.float32), lo, hi, legal, k, order)
    out = subset_attention(q_main, K, V, rows, scale)
    return {"z": z, "z_bits": z_bits, "u": u, "scores": scores, "rows": rows, "out": out, "lo": lo, "hi": hi, "k": k,
            "S": S}
