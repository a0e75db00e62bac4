"""The reference package's comparison helpers that this package also exports (src/attention_lab/__init__.py:14-32,
reference.py:41-97, indexer.py:57-64, metal_score.py:344-350, metal_attend.py:262-273): on the CPU, against the float64
oracle. They are explicit-math checks, not read paths, so no GPU is involved; the bf16 tolerance of a bf16 input is
the bf16 contract bar of the reference's tests (atol 5e-2), float64 inputs agree to 1e-12."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import attention_lab
from attention_lab import hip_attend, hip_score
from attention_lab.indexer import GroupedIndexer
from attention_lab.reference import dense_mask_reference, dense_reference, selection_mask
from oracle import exact

RNG = np.random.default_rng(5)


def t64(*shape):
    return torch.from_numpy(RNG.standard_normal(shape))


def test_import_surface_matches_the_reference():
    for name in ("dense_reference", "dense_mask_reference", "subset_attention", "flatten_cache", "gather_attention",
                 "gather_rows", "row_offsets", "FULL_BACKENDS", "full_attention", "GroupedIndexer", "candidate_scores",
                 "project_keys", "project_queries", "DecodeRequest", "dense_decode_step", "gathered_decode_step_kernel",
                 "prepare_request", "select_rows_kernel", "select_rows_recent", "select_rows_uniform",
                 "sparse_decode_step", "sparse_decode_step_kernel", "FIXED_PREFIX", "FIXED_RECENT", "SelectionLayout",
                 "fixed_budget", "legal_length", "selection_layout"):
        assert name in attention_lab.__all__ and hasattr(attention_lab, name), name


def test_dense_reference_decode_and_causal_chunk():
    B, G, h, C, d, L = 2, 3, 2, 40, 16, 33
    k, v = t64(B, G, C, d), t64(B, G, C, d)
    q1 = t64(B, G, h, 1, d)
    got = dense_reference(q1, k, v, valid_length=L).numpy()[:, :, :, 0]
    np.testing.assert_allclose(got, exact.dense_attention(q1.numpy()[:, :, :, 0], k.numpy(), v.numpy(), L),
                               rtol=1e-12, atol=1e-12)
    q5 = t64(B, G, h, 5, d)
    for qp in (None, [3, 10, 20, 31, 32]):
        got = dense_reference(q5, k, v, valid_length=L, query_positions=qp).numpy()
        want = exact.causal_attention(q5.numpy(), k.numpy(), v.numpy(), L, query_positions=qp)
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    with pytest.raises(ValueError):
        dense_reference(q1, k, v, valid_length=C + 1)


def test_dense_mask_reference_is_the_listed_subset():
    B, G, h, C, d, L = 2, 2, 3, 50, 16, 45
    k, v, q = t64(B, G, C, d), t64(B, G, C, d), t64(B, G, h, 1, d)
    rows = np.stack([np.stack([RNG.choice(L, size=9, replace=False) for _ in range(G)]) for _ in range(B)])
    got = dense_mask_reference(q, k, v, torch.from_numpy(rows), valid_length=L).numpy()[:, :, :, 0]
    want = exact.subset_attention(q.numpy()[:, :, :, 0], k.numpy(), v.numpy(), rows)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    valid = torch.ones(B, G, 9, dtype=torch.bool)
    valid[..., :3] = False                                              # dropped slots are not read
    got = dense_mask_reference(q, k, v, torch.from_numpy(rows), valid, valid_length=L).numpy()[:, :, :, 0]
    want = exact.subset_attention(q.numpy()[:, :, :, 0], k.numpy(), v.numpy(), np.where(valid.numpy(), rows, -1))
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    assert selection_mask(torch.from_numpy(rows), L).sum() == B * G * 9
    with pytest.raises(ValueError):
        dense_mask_reference(q, k, v, torch.full((B, G, 3), L), valid_length=L)   # outside the legal range


def test_bf16_inputs_stay_within_the_bf16_bar():
    B, G, h, C, d = 1, 2, 2, 64, 128
    k, v, q = (t64(*s).to(torch.bfloat16) for s in ((B, G, C, d), (B, G, C, d), (B, G, h, 1, d)))
    got = dense_reference(q, k, v).float().numpy()[:, :, :, 0]
    want = exact.dense_attention(q.double().numpy()[:, :, :, 0], k.double().numpy(), v.double().numpy(), C)
    assert got.dtype == np.float32 and np.abs(got - want).max() <= 5e-2


def test_grouped_indexer_reference_scores():
    G, h, d, r, B, T, C = 2, 2, 16, 8, 2, 3, 20
    idx = GroupedIndexer(G, h, d, r, dtype=torch.float64, seed=4)
    q_pre, k_pre = t64(B, G, h, T, d), t64(B, G, C, d)
    got = idx.reference_scores(q_pre, k_pre, 2, 17).numpy()
    for t in range(T):
        u = exact.grouped_u(q_pre[:, :, :, t].reshape(B, G, h * d).numpy(), idx.wq_t_scaled.numpy())
        zT = exact.project_keys(k_pre.numpy(), idx.wk.numpy())
        np.testing.assert_allclose(got[:, :, t], exact.grouped_scores(u, zT, 2, 17), rtol=1e-10, atol=1e-12)


def test_metal_module_reference_helpers():
    G, h, d, r, C, S = 3, 2, 128, 32, 60, 11
    zT, k_new, wk = t64(G, r, C), t64(G, d), t64(G, r, d)
    q_cat, wq_t = t64(G, h * d), t64(G, h * d, r)
    u, z_new, s = hip_score.reference_scores(zT, k_new, wk, q_cat, wq_t, 4, 50)
    u64 = exact.grouped_u(q_cat.numpy(), wq_t.numpy())
    np.testing.assert_allclose(u.numpy(), u64, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(z_new.numpy(), exact.z_column(k_new.numpy(), wk.numpy())[0], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(s.numpy(), exact.grouped_scores(u64, zT.numpy(), 4, 50), rtol=1e-3, atol=1e-3)
    K, V, q = t64(G, C, d), t64(G, C, d), t64(G, h, d)
    rows = torch.from_numpy(np.stack([RNG.choice(C, size=S, replace=False) for _ in range(G)]).astype(np.int32))
    got = hip_attend.reference_attend(K, V, q, rows).numpy()
    want = exact.subset_attention(q.numpy()[None], K.numpy()[None], V.numpy()[None], rows.numpy()[None].astype(np.int64))[0]
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_subset_attention_names_its_narrower_contract():
    """subset_attention runs only on the HIP attend kernel (bfloat16, d = 128, h*T <= 8 query rows per group): other
    inputs are refused up front with a ValueError that names the restriction, before any device work."""
    from attention_lab.sparse import subset_attention
    bf = torch.bfloat16
    q, ks = torch.zeros(1, 2, 2, 1, 128, dtype=bf), torch.zeros(1, 2, 5, 128, dtype=bf)
    with pytest.raises(ValueError, match="bfloat16 only; q is torch.float32"):
        subset_attention(q.float(), ks, ks)
    with pytest.raises(ValueError, match="bfloat16 only; k_sub is torch.float16"):
        subset_attention(q, ks.half(), ks.half())
    with pytest.raises(ValueError, match="head_dim 128 only, got 64"):
        subset_attention(torch.zeros(1, 2, 2, 1, 64, dtype=bf), torch.zeros(1, 2, 5, 64, dtype=bf),
                         torch.zeros(1, 2, 5, 64, dtype=bf))
    with pytest.raises(ValueError, match="h\\*T <= 8 query rows per group, got 16"):
        subset_attention(torch.zeros(1, 2, 8, 2, 128, dtype=bf), ks, ks, backend="explicit")
    with pytest.raises(ValueError, match="unknown subset backend"):
        subset_attention(q, ks, ks, backend="flash")
