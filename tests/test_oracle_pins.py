"""Pins of the CPU oracle (and of the host-side selection rules) - no GPU needed.

Each check is chosen so that a plausible slip in the oracle (a dropped term, a swapped index, a transposed operand,
the wrong tie order, renumbered rows) makes it fail; the `planted` tests prove that by running mutated copies of the
oracle functions against the same checks.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from attention_lab import selection as sel
from attention_lab.decode import prepare_request
from oracle import bf16, exact, ref_path, rules

RNG = np.random.default_rng(1234)


# ---------------------------------------------------------------------------------------------------------------------
# selection rules: the reference tests' known answers (test_attention_contracts.py:309-347, 237-239, 262;
# test_qwen_wrapper.py:387-392), checked on the oracle and on the product's host module
# ---------------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("budget,layout,legal", [(rules.budget, rules.layout, rules.legal),
                                                  (sel.fixed_budget, None, sel.legal_length)])
def test_selection_known_answers(budget, layout, legal):
    assert [budget(8192, 1 / 32), budget(8192, 1 / 8), budget(32768, 1 / 32)] == [256, 1024, 1024]
    assert [budget(100, 1 / 32), budget(50, 0.5), budget(4, 1.0)] == [3, 0, 0]
    assert budget(101, 1 / 8) == 13
    assert (legal(5, 10), legal(20, 10)) == (6, 10)
    for bad in ((-1, 10), (3, 0)):
        with pytest.raises(ValueError):
            legal(*bad)
    for bad_rho in (-0.1, 1.1, float("nan")):
        with pytest.raises(ValueError):
            budget(100, bad_rho)
    if layout is not None:
        assert layout(100) == (4, 36)
        assert layout(50) == (4, 4) and rules.step(50, 10) == (4, 4, 0, 50)
        assert layout(3) == (3, 3)
        assert rules.fixed_positions(100) == list(range(4)) + list(range(36, 100))
        assert rules.step(256, budget(256, 1 / 8))[:3] == (4, 192, 32)
        assert rules.step(128, budget(128, 1 / 8))[2:] == (16, 84)


def test_product_layout_known_answers():
    lay = sel.selection_layout(100)
    assert (lay.fixed_count, lay.candidate_count, lay.candidate_lo, lay.candidate_hi) == (68, 32, 4, 36)
    assert lay.fixed_positions() == list(range(4)) + list(range(36, 100))
    assert (sel.selection_layout(50).fixed_count, sel.selection_layout(50).candidate_count) == (50, 0)
    assert (sel.selection_layout(3).fixed_count, sel.selection_layout(3).fixed_prefix) == (3, 3)
    with pytest.raises(ValueError):
        sel.selection_layout(0)
    shrunk = prepare_request(1, 2, 128, valid_length=100, query_position=99, rho=1 / 32, device="cpu", n0=8192)
    assert (shrunk.k0, shrunk.k, shrunk.selected_count) == (256, 32, 100)
    only_f = prepare_request(1, 2, 128, valid_length=128, query_position=127, rho=0.0, device="cpu")
    assert (only_f.k, only_f.selected_count) == (0, 68)
    short = prepare_request(1, 2, 128, valid_length=60, query_position=59, rho=1 / 8, device="cpu")
    assert (short.k, short.selected_count) == (0, 60)
    r128 = prepare_request(1, 2, 128, valid_length=128, query_position=127, rho=1 / 8, device="cpu")
    assert (r128.layout.fixed_count, r128.k, r128.selected_count) == (68, 16, 84)
    assert r128.fixed_positions[0, 0].tolist() == list(range(4)) + list(range(64, 128))
    assert torch.equal(r128.fixed_rows - r128.offsets, r128.fixed_positions)
    assert torch.equal(r128.off_lo, r128.offsets + 4)
    with pytest.raises(ValueError):
        prepare_request(1, 2, 128, valid_length=0, query_position=0, rho=1 / 8, device="cpu")


def test_rules_agree_with_product_on_a_sweep():
    for n in list(range(1, 300)) + [2047, 2048, 8192, 32768, 131072]:
        lay = sel.selection_layout(n)
        assert rules.layout(n) == (lay.candidate_lo, lay.candidate_hi)
        for rho in (0.0, 1 / 32, 1 / 8, 0.5, 1.0):
            assert rules.budget(n, rho) == sel.fixed_budget(n, rho)


# ---------------------------------------------------------------------------------------------------------------------
# bf16 packing: known bit patterns
# ---------------------------------------------------------------------------------------------------------------------
def test_bf16_rne_known_patterns():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 0.0, -0.0, np.inf, -np.inf, 3.0e38], dtype=np.float32)
    want = [0x3F80, 0x3F80, 0x3F82, 0xC020, 0x0000, 0x8000, 0x7F80, 0xFF80, 0x7F62]
    assert bf16.from_f32(x).tolist() == want
    assert np.isnan(bf16.to_f32(bf16.from_f32(np.array([np.nan], dtype=np.float32))))[0]
    t = torch.randn(1000)
    assert np.array_equal(bf16.from_f32(t.numpy()), bf16.from_torch(t.to(torch.bfloat16)))


# ---------------------------------------------------------------------------------------------------------------------
# score: closed forms
# ---------------------------------------------------------------------------------------------------------------------
def test_grouped_score_closed_forms():
    G, h, d, r, C = 3, 2, 8, 5, 40
    zT = RNG.standard_normal((2, G, r, C))
    # a unit query picks one table row: u = e_j when q_cat = e_f and wq_t[g, f, :] = e_j
    q_cat = np.zeros((2, G, h * d))
    wq_t = np.zeros((G, h * d, r))
    for g in range(G):
        q_cat[:, g, 3 + g] = 1.0
        wq_t[g, 3 + g, (g + 1) % r] = 1.0
    u = exact.grouped_u(q_cat, wq_t)
    s = exact.grouped_scores(u, zT, 7, 30)
    for g in range(G):
        np.testing.assert_array_equal(s[:, g], zT[:, g, (g + 1) % r, 7:30])
    # linearity in u and the scanned range only
    u2 = RNG.standard_normal((2, G, r))
    np.testing.assert_allclose(exact.grouped_scores(2 * u2, zT, 0, C), 2 * exact.grouped_scores(u2, zT, 0, C))
    poisoned = zT.copy()
    poisoned[..., :7] = np.nan
    poisoned[..., 30:] = np.nan
    assert np.isfinite(exact.grouped_scores(u2, poisoned, 7, 30)).all()


def test_z_column_closed_form():
    G, r, d = 2, 4, 6
    wk = np.zeros((G, r, d))
    for g in range(G):
        for j in range(r):
            wk[g, j, (j + g) % d] = 1.0
    k_new = RNG.standard_normal((3, G, d)).astype(np.float32).astype(np.float64)
    z, bits = exact.z_column(k_new, wk)
    for g in range(G):
        for j in range(r):
            np.testing.assert_array_equal(z[:, g, j], k_new[:, g, (j + g) % d])
    np.testing.assert_array_equal(bits, bf16.from_f32(z.astype(np.float32)))


def test_project_keys_pins():
    """exact.project_keys (indexer.py:15-17), the bulk index-table build both MFMA kernels are checked against: unit
    rows of wk pick one coordinate of every key, one column equals the separately written z_column of that key, a
    double loop over (g, j, t, e) agrees, and the table is laid out [B, G, r, T] (index dim before position)."""
    B, G, T, r, d = 2, 3, 7, 5, 6
    perm = np.array([[(j * 2 + g) % d for j in range(r)] for g in range(G)])
    wk = np.zeros((G, r, d))
    for g in range(G):
        for j in range(r):
            wk[g, j, perm[g, j]] = 1.0
    k_pre = RNG.standard_normal((B, G, T, d))
    zT = exact.project_keys(k_pre, wk)
    assert zT.shape == (B, G, r, T)
    for g in range(G):
        for j in range(r):
            np.testing.assert_array_equal(zT[:, g, j, :], k_pre[:, g, :, perm[g, j]])
    wk = RNG.standard_normal((G, r, d))
    zT = exact.project_keys(k_pre, wk)
    for t in range(T):
        z, _ = exact.z_column(k_pre[:, :, t, :], wk)
        np.testing.assert_allclose(zT[..., t], z, rtol=1e-13, atol=1e-13)
    loop = np.zeros((B, G, r, T))
    for b in range(B):
        for g in range(G):
            for j in range(r):
                for t in range(T):
                    loop[b, g, j, t] = sum(wk[g, j, e] * k_pre[b, g, t, e] for e in range(d))
    np.testing.assert_allclose(zT, loop, rtol=1e-12, atol=1e-12)


def test_lightning_reduces_to_grouped_and_relu_clamps():
    B, KG, L, r = 2, 3, 50, 32
    keys = RNG.standard_normal((B, KG, L, r))
    q = RNG.standard_normal((B, KG, 1, r))
    s_l = exact.lightning_scores(keys, q, np.ones((B, KG, 1)), 4, 40, relu=False)
    s_g = exact.grouped_scores(q[:, :, 0], keys.transpose(0, 1, 3, 2), 4, 40)
    np.testing.assert_allclose(s_l, s_g, rtol=1e-12, atol=1e-12)
    s_r = exact.lightning_scores(keys, q, np.ones((B, KG, 1)), 4, 40, relu=True)
    np.testing.assert_array_equal(s_r, np.maximum(s_g, 0.0))
    w = RNG.random((B, KG, 2))
    q2 = RNG.standard_normal((B, KG, 2, r))
    two = exact.lightning_scores(keys, q2, w, 0, L)
    one = [exact.lightning_scores(keys, q2[:, :, i:i + 1], w[:, :, i:i + 1], 0, L) for i in range(2)]
    np.testing.assert_allclose(two, one[0] + one[1])


def test_batched_lightning_is_one_single_query_score_per_query_with_a_causal_bound():
    B, KG, L, r, T, nh, lo, hi, p0 = 2, 2, 40, 32, 5, 2, 3, 37, 20
    keys = RNG.standard_normal((B, KG, L, r))
    q = RNG.standard_normal((B, KG, T, nh, r))
    w = RNG.random((B, KG, T, nh))
    full = exact.lightning_scores_batched(keys, q, w, lo, hi)
    causal = exact.lightning_scores_batched(keys, q, w, lo, hi, q_pos0=p0)
    for t in range(T):
        one = exact.lightning_scores(keys, q[:, :, t], w[:, :, t], lo, hi)
        np.testing.assert_allclose(full[:, :, t], one, rtol=1e-12, atol=1e-12)
        for m in range(lo, hi):   # the causal bound, element by element
            if m <= p0 + t:
                np.testing.assert_array_equal(causal[:, :, t, m - lo], full[:, :, t, m - lo])
            else:
                assert np.isnan(causal[:, :, t, m - lo]).all()
    # a unit query on head 0 with weight 1 (others weight 0) and no ReLU reads one key coordinate
    q1 = np.zeros((1, 1, 1, 1, r)); q1[..., 7] = 1.0
    s1 = exact.lightning_scores_batched(keys[:1, :1], q1, np.ones((1, 1, 1, 1)), 0, L, relu=False)
    np.testing.assert_array_equal(s1[0, 0, 0], keys[0, 0, :, 7])


# ---------------------------------------------------------------------------------------------------------------------
# top-k: brute force with planted ties, NaN and signed zeros
# ---------------------------------------------------------------------------------------------------------------------
def brute_topk(row, k):
    def key(i):
        v = float(row[i])
        return (1 if math.isnan(v) else 0, -(v + 0.0) if not math.isnan(v) else 0.0, i)
    return sorted(range(len(row)), key=key)[:k]


def test_topk_against_brute_force():
    for M in (1, 2, 7, 64, 333):
        s = RNG.integers(-3, 4, size=(5, M)).astype(np.float32) * 0.5   # many ties
        s[0, ::3] = np.nan
        s[1, ::2] = -0.0
        s[1, 1::2] = 0.0
        s[2, ::4] = -np.inf
        for k in sorted({0, 1, M // 3, M}):
            got = exact.topk(s, k, order="score")
            for i in range(5):
                assert got[i].tolist() == brute_topk(s[i], k)
            pos = exact.topk(s, k, order="position")
            assert np.array_equal(pos, np.sort(got, axis=-1))


def test_select_rows_layout():
    s = RNG.standard_normal((2, 3, 32)).astype(np.float32)
    lo, hi, legal, k = 4, 36, 100, 5
    r_score = exact.select_rows(s, lo, hi, legal, k, "score")
    r_pos = exact.select_rows(s, lo, hi, legal, k, "position")
    assert r_score.shape == (2, 3, 68 + 5)
    assert r_score[0, 0, :68].tolist() == list(range(4)) + list(range(36, 100))
    top = r_score[..., 68:] - lo
    assert np.array_equal(np.take_along_axis(s, top, -1), -np.sort(-s, -1)[..., :k])
    assert np.array_equal(r_pos, np.sort(r_score, -1))


# ---------------------------------------------------------------------------------------------------------------------
# attention: closed forms and two independent formulations
# ---------------------------------------------------------------------------------------------------------------------
def test_attention_closed_forms():
    B, G, h, d, C = 2, 3, 2, 16, 40
    q = RNG.standard_normal((B, G, h, d))
    K = RNG.standard_normal((B, G, C, d))
    V = RNG.standard_normal((B, G, C, d))
    one = np.full((B, G, 1), 17)
    np.testing.assert_allclose(exact.subset_attention(q, K, V, one), np.broadcast_to(V[:, :, 17:18], (B, G, h, d)))
    rows = np.stack([np.stack([RNG.permutation(C)[:9] for _ in range(G)]) for _ in range(B)])
    uniform = exact.subset_attention(np.zeros_like(q), K, V, rows)
    for b in range(B):
        for g in range(G):
            np.testing.assert_allclose(uniform[b, g], np.broadcast_to(V[b, g, rows[b, g]].mean(0), (h, d)))
    sub = exact.subset_attention(q, K, V, rows)
    np.testing.assert_allclose(sub, exact.dense_mask_attention(q, K, V, rows), atol=1e-12)
    np.testing.assert_allclose(sub, exact.subset_attention(q, K, V, rows[..., ::-1]), atol=1e-12)
    full = np.broadcast_to(np.arange(30), (B, G, 30))
    np.testing.assert_allclose(exact.subset_attention(q, K, V, full), exact.dense_attention(q, K, V, 30), atol=1e-12)
    padded = np.concatenate([rows, -np.ones((B, G, 3), dtype=rows.dtype)], -1)
    np.testing.assert_allclose(exact.subset_attention(q, K, V, padded), sub, atol=1e-12)
    scaled = exact.subset_attention(q * 2.0, K, V, rows, scale=0.5 / math.sqrt(d))
    np.testing.assert_allclose(scaled, sub, atol=1e-12)
    np.testing.assert_allclose(exact.dense_attention(q, K, V, 1), np.broadcast_to(V[:, :, :1], (B, G, h, d)))


def test_ref_path_matches_exact():
    """The reference's torch op sequence on the CPU agrees with the float64 oracle on tie-free inputs."""
    B, G, h, d, r, C, L = 2, 4, 2, 32, 8, 300, 290
    gen = torch.Generator().manual_seed(0)
    tt = lambda *s: torch.randn(*s, generator=gen, dtype=torch.float64)  # noqa: E731
    K, V, q, q_pre, k_new, zT = tt(B, G, C, d), tt(B, G, C, d), tt(B, G, h, 1, d), tt(B, G, h, 1, d), tt(B, G, 1, d), tt(B, G, r, C)
    wq_t, wk = tt(G, h * d, r) * 0.1, tt(G, r, d) * 0.1
    k0 = rules.budget(L, 1 / 8)
    z_before = zT.clone()
    out, rows = ref_path.sparse_layer_step(q, q_pre, K, V, zT, wq_t, wk, k_new, L, k0)
    e = exact.sparse_step(q.numpy()[:, :, :, 0], q_pre.numpy().reshape(B, G, h * d), K.numpy(), V.numpy(),
                          z_before.numpy(), wq_t.numpy(), wk.numpy(), k_new.numpy()[:, :, 0], L, k0)
    pos = (rows.view(B, G, -1) - (torch.arange(B * G) * C).view(B, G, 1)).numpy()
    assert np.array_equal(np.sort(pos, -1), np.sort(e["rows"], -1))
    np.testing.assert_allclose(out.numpy()[:, :, :, 0], e["out"], atol=1e-10)
    np.testing.assert_allclose(zT.numpy()[..., L - 1], e["z"], atol=1e-12)
    dense = ref_path.dense_layer_step(q, K, V, L)
    np.testing.assert_allclose(dense.numpy()[:, :, :, 0], exact.dense_attention(q.numpy()[:, :, :, 0], K.numpy(),
                                                                                   V.numpy(), L), atol=1e-10)


# ---------------------------------------------------------------------------------------------------------------------
# planted mistakes: mutated copies of the oracle must fail the checks above
# ---------------------------------------------------------------------------------------------------------------------
def test_planted_mistakes_are_caught():
    # 1. highest-index tie-break instead of lowest
    def topk_wrong_ties(scores, k):
        s = np.asarray(scores, dtype=np.float64)
        return np.array([np.lexsort((-np.arange(s.shape[-1]), -row))[:k] for row in s])
    s = np.array([[1.0, 2.0, 2.0, 0.5, 2.0]], dtype=np.float32)
    assert topk_wrong_ties(s, 2)[0].tolist() != brute_topk(s[0], 2)
    assert exact.topk(s, 2)[0].tolist() == brute_topk(s[0], 2)

    # 2. renumbered rows (positions replaced by 0..S-1) change the answer
    q = RNG.standard_normal((1, 1, 2, 8))
    K = RNG.standard_normal((1, 1, 20, 8))
    V = RNG.standard_normal((1, 1, 20, 8))
    rows = np.array([[[2, 9]]])
    assert np.abs(exact.subset_attention(q, K, V, rows) - exact.subset_attention(q, K, V, np.array([[[0, 1]]]))).max() > 1e-3

    # 3. a transposed weight operand breaks the unit-vector check of the score
    G, h, d, r = 2, 1, 4, 4
    q_cat = np.zeros((1, G, h * d))
    q_cat[:, :, 1] = 1.0
    wq_t = np.zeros((G, h * d, r))
    wq_t[:, 1, 3] = 1.0
    good = exact.grouped_u(q_cat, wq_t)
    bad = np.einsum("bgf,gjf->bgj", q_cat, wq_t)
    assert good[0, 0].tolist() == [0, 0, 0, 1] and bad[0, 0].tolist() != [0, 0, 0, 1]

    # 4. a softmax that drops the scale differs from the reference scale
    sub = exact.subset_attention(q, K, V, rows)
    assert np.abs(sub - exact.subset_attention(q, K, V, rows, scale=1.0)).max() > 1e-4

    # 5. a bulk index-table build with its output axes transposed ([B, G, T, r]) or contracting the wrong weight axis
    #    fails project_keys' unit-row check
    Gk, rk, dk, Tk = 1, 3, 3, 4
    wk = np.zeros((Gk, rk, dk))
    wk[0, 0, 2] = wk[0, 1, 0] = wk[0, 2, 1] = 1.0
    k_pre = RNG.standard_normal((1, Gk, Tk, dk))
    want = np.stack([k_pre[0, 0, :, 2], k_pre[0, 0, :, 0], k_pre[0, 0, :, 1]])
    np.testing.assert_array_equal(exact.project_keys(k_pre, wk)[0, 0], want)
    transposed_out = np.einsum("gjd,bgtd->bgtj", wk, k_pre)
    wrong_axis = np.einsum("gdj,bgtd->bgjt", wk, k_pre)
    assert transposed_out[0, 0].shape != want.shape or not np.array_equal(transposed_out[0, 0], want)
    assert not np.array_equal(wrong_axis[0, 0], want)


def test_causal_attention_is_one_dense_read_per_query():
    """The masked formulation of the prefill read equals, query by query, the sliced dense read over the first
    min(position + 1, valid_length) keys; a single last-position query is exactly dense_attention."""
    rng = np.random.default_rng(11)
    B, G, h, T, d, C = 2, 3, 2, 5, 16, 40
    q = rng.standard_normal((B, G, h, T, d))
    K, V = rng.standard_normal((B, G, C, d)), rng.standard_normal((B, G, C, d))
    for L, qp in ((30, None), (30, [0, 7, 29, 29, 35]), (40, [3, 3, 12, 39, 1])):
        got = exact.causal_attention(q, K, V, L, qp)
        pos = list(range(L - T, L)) if qp is None else qp
        for t, p in enumerate(pos):
            want = exact.dense_attention(q[:, :, :, t], K, V, min(p + 1, L))
            np.testing.assert_allclose(got[:, :, :, t], want, atol=1e-12)
    np.testing.assert_allclose(exact.causal_attention(q[:, :, :, :1], K, V, 30)[:, :, :, 0],
                               exact.dense_attention(q[:, :, :, 0], K, V, 30), atol=1e-12)
    first = exact.causal_attention(q, K, V, 30, [0, 0, 0, 0, 0])          # position 0 reads only key 0
    np.testing.assert_allclose(first, np.broadcast_to(V[:, :, None, None, 0], first.shape), atol=1e-12)
