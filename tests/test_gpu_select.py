"""Top-k / row-list kernel on the GPU against the oracle's deterministic top-k: index sets and orders bit-exact.

The reference uses torch.topk (decode.py:86-93) and checks only set equality against a float64 brute force on tie-free
scores (test_attention_contracts.py:254-277). Given identical fp32 scores, this kernel must return exactly the oracle's
indices, including the order contract for ties (lower index first), NaN (never before a number) and -0.0 == +0.0.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from attention_lab import hip_select
from oracle import exact

pytestmark = pytest.mark.gpu


def heavy_tail(R, M, seed, frac=0.02, sigma=3.0):
    """Config 2 scores: N(0,1) with 2% of positions lifted by +3 sigma (seeded)."""
    rng = np.random.default_rng(seed)
    s = rng.standard_normal((R, M)).astype(np.float32)
    n = max(1, int(frac * M))
    for i in range(R):
        idx = rng.choice(M, size=n, replace=False)
        s[i, idx] += np.float32(sigma * s[i].std())
    return s


def check_topk(gpu, s: np.ndarray, k: int):
    """Both selections (one workgroup per row; histogram + classify + resolve over the chip) against the oracle."""
    t = torch.from_numpy(s).to(gpu)
    for order in ("score", "position"):
        want = exact.topk(s, k, order=order)
        for tiled in (False, True):
            vals, idx = hip_select.topk(t, k, order=order, tiled=tiled)
            torch.cuda.synchronize()
            got = idx.cpu().numpy()
            assert np.array_equal(got, want), f"order={order} M={s.shape[-1]} k={k} tiled={tiled}: indices differ"
            np.testing.assert_array_equal(vals.cpu().numpy(), np.take_along_axis(s, want, -1))


@pytest.mark.parametrize("M", [1, 5, 100, 1000, 4093, 32700, 32768, 40000, 65468, 131008])
def test_topk_matches_oracle_heavy_tail(gpu, M):
    R = 4 if M > 40000 else 8
    s = heavy_tail(R, M, seed=M)
    for k in sorted({0, 1, max(1, M // 32), min(M, 4096), M}):
        check_topk(gpu, s, k)


@pytest.mark.parametrize("M,k", [(32700, 1024), (65468, 2046), (131008, 4094)])
def test_topk_position_order_large_k(gpu, M, k):
    s = heavy_tail(2, M, seed=k)
    t = torch.from_numpy(s).to(gpu)
    _, idx = hip_select.topk(t, k, order="position")
    torch.cuda.synchronize()
    assert np.array_equal(idx.cpu().numpy(), exact.topk(s, k, order="position"))


@pytest.mark.parametrize("M,k", [(20000, 6000), (70000, 8192)])
def test_score_order_beyond_4096(gpu, M, k):
    """Score order sorts up to 8192 selected pairs in LDS (both selections)."""
    check_topk(gpu, heavy_tail(2, M, seed=k), k)


@pytest.mark.parametrize("M,k,gen", [(5000, 1025, "ties"), (9000, 2049, "specials"), (40000, 4096, "ties"),
                                     (3000, 2048, "zeros"), (70000, 3000, "normal")])
def test_score_order_sorts_of_two_to_four_thousand(gpu, M, k, gen):
    """Score order with 1024 < k <= 4096: the LDS radix sort over two to four sub-blocks of 1024 pairs (digit counts,
    then per sub-block offsets); ties stay in index order, NaN last, -0.0 == +0.0."""
    rng = np.random.default_rng(M + k)
    R = 3
    s = {"normal": lambda: heavy_tail(R, M, seed=k), "ties": lambda: tie_heavy(rng, (R, M)),
         "specials": lambda: specials(rng, (R, M)), "zeros": lambda: np.zeros((R, M), np.float32)}[gen]()
    check_topk(gpu, s, k)


@pytest.mark.parametrize("M,k,gen", [(32700, 16384, "normal"), (40000, 20000, "normal"), (32768, 32768, "normal"),
                                     (20000, 9000, "ties"), (12000, 10000, "specials"), (10000, 9000, "zeros"),
                                     (300000, 9000, "normal")])
def test_score_order_past_the_lds_sort(gpu, M, k, gen):
    """Score order with k > 8192: the position-order select, then the stable radix pass; ties stay in index order,
    NaN last, -0.0 == +0.0; the compact, bitmap and single-workgroup (M > 262144) selects all feed it."""
    rng = np.random.default_rng(M + k)
    R = 2
    s = {"normal": lambda: heavy_tail(R, M, seed=k), "ties": lambda: tie_heavy(rng, (R, M)),
         "specials": lambda: specials(rng, (R, M)), "zeros": lambda: np.zeros((R, M), np.float32)}[gen]()
    check_topk(gpu, s, k)


def test_ties_resolve_to_the_lowest_index(gpu):
    rng = np.random.default_rng(7)
    for M, levels in ((1000, 3), (5000, 17), (32700, 50)):
        s = (rng.integers(0, levels, size=(6, M)) * 0.5).astype(np.float32)
        s[0] = 1.0                                                   # every score equal
        for k in (1, 7, M // 32, M // 2):
            check_topk(gpu, s, k)


def test_nan_signed_zero_and_infinities(gpu):
    rng = np.random.default_rng(3)
    M = 3000
    s = rng.standard_normal((4, M)).astype(np.float32)
    s[0, ::7] = np.nan
    s[1, :] = 0.0
    s[1, ::2] = -0.0                                                 # -0.0 ties with +0.0 by index
    s[2, ::5] = np.inf
    s[2, 1::5] = -np.inf
    s[3, :] = np.nan
    s[3, 10:20] = -np.inf
    for k in (1, 50, 500, M - 1, M):
        for order in ("score", "position"):
            if k > 4096:
                continue
            t = torch.from_numpy(s).to(gpu)
            for tiled in (False, True):
                _, idx = hip_select.topk(t, k, order=order, tiled=tiled)
                torch.cuda.synchronize()
                assert np.array_equal(idx.cpu().numpy(), exact.topk(s, k, order=order)), (k, order, tiled)


@pytest.mark.parametrize("legal,k0,order", [(2048, 64, "position"), (2048, 64, "score"), (300, 37, "score"),
                                            (60, 10, "position"), (32768, 1024, "position"), (32768, 1024, "score"),
                                            (100, 0, "score"), (1000, 932, "position"), (32768, 16384, "score"),
                                            (32768, 32700, "score"), (20000, 9000, "score")])
def test_select_rows_matches_oracle(gpu, legal, k0, order):
    from oracle import rules
    B, G = 2, 8
    lo, hi, k, S = rules.step(legal, k0)
    C = legal + 40
    s = heavy_tail(B * G, max(hi - lo, 1), seed=legal + k0)[:, :hi - lo].reshape(B, G, hi - lo)
    t = torch.from_numpy(np.ascontiguousarray(s)).to(gpu)
    rows, flat = hip_select.select_rows(t, lo, hi, legal, k, C, order=order, want_flat=True)
    torch.cuda.synchronize()
    want = exact.select_rows(s, lo, hi, legal, k, order=order)
    assert rows.shape == (B, G, S)
    assert np.array_equal(rows.cpu().numpy(), want)
    off = (np.arange(B * G) * C).reshape(B, G, 1)
    assert np.array_equal(flat.cpu().numpy().reshape(B, G, S), want + off)


@pytest.mark.parametrize("B,C,L,order,tiled,rho", [(1, 2048 + 64, 2048, "position", True, 1 / 32),
                                                   (4, 32768, 32768, "score", True, 1 / 32),
                                                   (2, 70000, 70000, "position", True, 1 / 32),
                                                   (3, 1000, 777, "score", True, 1 / 32),
                                                   (2, 32768, 32768, "position", False, 1 / 32),
                                                   (2, 140000, 140000, "position", True, 1 / 32),
                                                   (2, 32768, 32768, "score", True, 1 / 2),
                                                   (1, 40000, 40000, "score", True, 1 / 4)])
def test_histogram_handoff_from_the_score_kernel(gpu, B, C, L, order, tiled, rho):
    """score_grouped(state=) + select_rows(state=) gives exactly the rows of the self-contained select, leaves the
    state zeroed, and stays exact over repeated calls on fresh data (a stale histogram would break it)."""
    from attention_lab import _native as nat
    from attention_lab import hip_score
    from oracle import rules
    G, r = 8, 32
    lo, hi, k, S = rules.step(L, rules.budget(L, rho))
    state = torch.zeros(B, G, nat.SELECT_STATE_WORDS, dtype=torch.int32, device=gpu)
    for rep in range(3):
        gen = torch.Generator().manual_seed(100 * rep + B)
        zT = torch.randn(B, G, r, C, generator=gen).to(torch.bfloat16).to(gpu)
        u = torch.randn(B, G, r, generator=gen).to(gpu)
        s = hip_score.score_grouped(zT, lo, hi, u=u, state=state)
        rows_h, _ = hip_select.select_rows(s, lo, hi, L, k, C, order=order, state=state, tiled=tiled)
        torch.cuda.synchronize()
        assert int(state.abs().sum()) == 0, "the select kernels must leave the state zeroed"
        rows_p, _ = hip_select.select_rows(s, lo, hi, L, k, C, order=order)
        torch.cuda.synchronize()
        assert torch.equal(rows_h, rows_p)
        want = exact.select_rows(s.cpu().numpy(), lo, hi, L, k, order=order)
        assert np.array_equal(rows_h.cpu().numpy(), want)


def score_keys(s):
    """Order-preserving uint32 keys of fp32 scores: NaN -> 0, -0.0 -> +0.0, negative -> bitwise not, else sign set."""
    u = np.ascontiguousarray(s, dtype=np.float32).view(np.uint32).copy()
    u[u == 0x80000000] = 0
    key = np.where(u & 0x80000000, ~u, u | 0x80000000).astype(np.uint32)
    key[np.isnan(s)] = 0
    return key


def state_for(s):
    """Select state [B, G, 2112] of the scores: the histogram of their first 11-bit digit, then its 64 sums of 32
    consecutive bins (what the score kernel leaves for the select)."""
    from attention_lab import _native as nat
    B, G, M = s.shape
    st = np.zeros((B, G, nat.SELECT_STATE_WORDS), dtype=np.int64)
    d = (score_keys(s) >> 21).astype(np.int64)
    for b in range(B):
        for g in range(G):
            st[b, g, :2048] = np.bincount(d[b, g], minlength=2048)
    st[..., 2048:2112] = st[..., :2048].reshape(B, G, 64, 32).sum(-1)
    return torch.from_numpy(st.astype(np.int32))


@pytest.mark.parametrize("B,C,lo,hi,fused", [(2, 32768, 4, 32704, True), (2, 32768, 4, 32704, False),
                                             (1, 3000, 4, 2900, True), (3, 1000, 0, 1000, False)])
def test_score_kernel_hands_over_the_first_digit_histogram(gpu, B, C, lo, hi, fused):
    """The state the score kernel leaves is exactly the histogram of its own scores' first 11-bit digits (counted
    once per score, whatever the workgroup split) followed by its 64 super-bin sums."""
    from attention_lab import _native as nat
    from attention_lab import hip_score
    from attention_lab.indexer import GroupedIndexer
    G, r, h, d = 8, 32, 4, 128
    gen = torch.Generator().manual_seed(B * 7 + C)
    zT = torch.randn(B, G, r, C, generator=gen).to(torch.bfloat16).to(gpu)
    state = torch.zeros(B, G, nat.SELECT_STATE_WORDS, dtype=torch.int32, device=gpu)
    if fused:
        idx = GroupedIndexer(G, h, d, r, device=gpu, dtype=torch.bfloat16, seed=3)
        q_cat = torch.randn(B, G, h * d, generator=gen).to(torch.bfloat16).to(gpu)
        s = hip_score.score_grouped(zT, lo, hi, q_cat=q_cat, wq_t=idx.wq_t_scaled, state=state)
    else:
        u = torch.randn(B, G, r, generator=gen).to(gpu)
        s = hip_score.score_grouped(zT, lo, hi, u=u, state=state)
    torch.cuda.synchronize()
    assert torch.equal(state.cpu(), state_for(s.cpu().numpy()))


@pytest.mark.parametrize("G,C,lo,hi,fused", [(3, 32256, 4, 32000, False), (5, 20000, 4, 19500, True),
                                             (1, 9000, 0, 8999, False)])
def test_histogram_is_exact_when_a_row_spans_the_xcds(gpu, G, C, lo, hi, fused):
    """Grids that are not a multiple of 8 keep the hardware's round-robin order, so the workgroups of one row run on
    different XCDs (each with its own L2) and their histogram atomics meet only in memory: the state must still be
    exactly the histogram of the scores."""
    from attention_lab import _native as nat
    from attention_lab import hip_score
    from attention_lab.indexer import GroupedIndexer
    B, r, h, d = 1, 32, 2, 128
    gen = torch.Generator().manual_seed(G * 11 + C)
    zT = torch.randn(B, G, r, C, generator=gen).to(torch.bfloat16).to(gpu)
    state = torch.zeros(B, G, nat.SELECT_STATE_WORDS, dtype=torch.int32, device=gpu)
    for rep in range(3):
        state.zero_()
        if fused:
            idx = GroupedIndexer(G, h, d, r, device=gpu, dtype=torch.bfloat16, seed=rep)
            q_cat = torch.randn(B, G, h * d, generator=gen).to(torch.bfloat16).to(gpu)
            s = hip_score.score_grouped(zT, lo, hi, q_cat=q_cat, wq_t=idx.wq_t_scaled, state=state)
        else:
            u = torch.randn(B, G, r, generator=gen).to(gpu)
            s = hip_score.score_grouped(zT, lo, hi, u=u, state=state)
        torch.cuda.synchronize()
        assert torch.equal(state.cpu(), state_for(s.cpu().numpy())), f"rep {rep}"


def tie_heavy(rng, shape):
    return rng.integers(0, 6, size=shape).astype(np.float32) * 0.25


def specials(rng, shape):
    s = rng.standard_normal(shape).astype(np.float32)
    m = rng.random(shape)
    s[m < 0.05] = np.nan
    s[(m >= 0.05) & (m < 0.1)] = -0.0
    s[(m >= 0.1) & (m < 0.15)] = 0.0
    s[(m >= 0.15) & (m < 0.17)] = np.inf
    s[(m >= 0.17) & (m < 0.19)] = -np.inf
    return s


@pytest.mark.parametrize("M,k,gen", [(1, 1, "normal"), (3, 2, "normal"), (1000, 31, "normal"), (1024, 1024, "normal"),
                                     (1025, 32, "normal"), (4096, 128, "normal"), (4097, 129, "normal"),
                                     (8191, 4000, "normal"), (32704, 1024, "normal"), (32768, 1024, "normal"),
                                     (32769, 1025, "normal"), (70000, 2187, "ties"), (131072, 4096, "normal"),
                                     (262145, 8192, "normal"), (70000, 2187, "normal"),
                                     (3000, 100, "ties"), (32704, 1024, "ties"), (20000, 600, "specials"),
                                     (32704, 32704, "normal"), (5000, 4999, "ties")])
def test_tiled_select_matches_the_oracle(gpu, M, k, gen):
    """Tiled select (4096-key tiles classified, one workgroup per row resolves) vs the oracle: plain, ties at the
    threshold (taken in index order), more than 8192 candidates sharing the threshold's first digit (streaming
    fallback), NaN / +-0 / +-inf, k = M, long rows, a row too long for the tiled path (262144 < M); the state is left
    zeroed and a second call on other data is exact too."""
    rng = np.random.default_rng(M + k)
    B, G = 2, 3
    lo = 5
    hi = lo + M
    legal = hi + 7
    C = legal + 3
    state = None
    for rep in range(2):
        shape = (B, G, M)
        s = {"normal": lambda: rng.standard_normal(shape).astype(np.float32),
             "ties": lambda: tie_heavy(rng, shape), "specials": lambda: specials(rng, shape)}[gen]()
        st = state_for(s).to(gpu)
        if state is None:
            state = st
        else:
            assert int(state.abs().sum()) == 0
            state.copy_(st)
        t = torch.from_numpy(s).to(gpu)
        rows, flat = hip_select.select_rows(t, lo, hi, legal, k, C, order="position", want_flat=True, state=state)
        torch.cuda.synchronize()
        want = exact.select_rows(s, lo, hi, legal, k, order="position")
        assert np.array_equal(rows.cpu().numpy(), want), f"rep {rep}"
        off = (np.arange(B * G) * C).reshape(B, G, 1)
        assert np.array_equal(flat.cpu().numpy().reshape(B, G, -1), want + off)
        assert int(state.abs().sum()) == 0, "the select must leave the state zeroed"


def test_validation(gpu):
    t = torch.zeros(2, 100, device=gpu)
    with pytest.raises(ValueError):
        hip_select.topk(t, 101)
    with pytest.raises(ValueError):
        hip_select.topk(t.double(), 3)
    with pytest.raises(ValueError):
        hip_select.topk(t, 3, order="random")
    with pytest.raises(ValueError):
        hip_select.select_rows(torch.zeros(1, 8, 10, device=gpu), 4, 15, 20, 3, 32)   # M != hi - lo
