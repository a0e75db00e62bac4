"""Gather-free attend and dense decode kernels against the oracle (contracts of tests/test_metal_attend.py).

Preset tolerances (test_metal_attend.py:28-29): fp32 output vs the float64 masked-dense reference on the same bf16
inputs, max |d| <= 5e-5 and relative norm <= 1e-5, for every partition count; the bf16 output within one bf16 ulp of
the RNE of the fp32 output, >= 99% bitwise. north_star's looser bf16 bound (max 2e-2, mean 2e-3) is implied.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from attention_lab import hip_attend
from attention_lab.decode import prepare_request
from attention_lab.full import full_attention
from oracle import bf16, exact

pytestmark = pytest.mark.gpu
TOL = {"out_atol": 5e-5, "out_rel_norm": 1e-5, "bf16_ulp": 2.0 ** -8}
PARTS = (1, 2, 4, 8, 16, 32, 64)
f64 = bf16.values


def make(gpu, G=8, h=2, d=128, C=2304, seed=0, B=1):
    gen = torch.Generator().manual_seed(seed)
    K4 = torch.randn(B, G, C, d, generator=gen).to(torch.bfloat16)
    V4 = torch.randn(B, G, C, d, generator=gen).to(torch.bfloat16)
    q5 = torch.randn(B, G, h, 1, d, generator=gen).to(torch.bfloat16)
    return K4.to(gpu), V4.to(gpu), q5.to(gpu)


def row_list(G, C, L, rho, seed=0, B=1):
    """F plus k distinct random candidates per group (the shape of a D selection), int64 [B, G, S]."""
    req = prepare_request(1, G, C, valid_length=L, query_position=L - 1, rho=rho, device="cpu")
    gen = torch.Generator().manual_seed(seed)
    lo, hi, k = req.layout.candidate_lo, req.layout.candidate_hi, req.k
    fixed = torch.tensor(req.layout.fixed_positions(), dtype=torch.long)
    rows = [torch.cat([fixed, lo + torch.randperm(hi - lo, generator=gen)[:k]]) for _ in range(B * G)]
    return torch.stack(rows).view(B, G, -1), req


def ref_of(q5, K4, V4, rows3):
    q = f64(q5)[:, :, :, 0, :]
    return exact.dense_mask_attention(q, f64(K4), f64(V4), rows3.numpy())


def check(out, ref, what, atol=TOL["out_atol"]):
    o = f64(out).reshape(ref.shape)
    diff = float(np.abs(o - ref).max())
    rel = float(np.linalg.norm(o - ref) / np.linalg.norm(ref))
    assert diff <= atol, f"{what}: max abs diff {diff:.3e}"
    assert rel <= TOL["out_rel_norm"] * max(1.0, atol / TOL["out_atol"]), f"{what}: rel norm {rel:.3e}"


@pytest.mark.parametrize("C,L,rho", [(2304, 2176 + 65, 1 / 8), (2304, 400, 1 / 32), (2304, 300, 1 / 8),
                                     (2304, 73, 1.0)])
def test_matches_dense_mask_reference_for_every_partition_count(gpu, C, L, rho):
    ma = hip_attend.HipAttend()
    K4, V4, q5 = make(gpu, C=C)
    rows3, req = row_list(8, C, L, rho)
    assert rows3.shape[-1] == req.selected_count
    K, V, q, rows = hip_attend.model_views(K4, V4, q5, rows3.to(gpu))
    ref = ref_of(q5, K4, V4, rows3)[0]
    for P in PARTS:
        out = ma(K, V, q, rows, partitions=P)
        ob = ma(K, V, q, rows, partitions=P, out_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        check(out, ref, f"P={P}")
        rne = out.to(torch.bfloat16).float().cpu()
        tol = TOL["bf16_ulp"] * rne.abs() + 1e-7
        assert bool(((ob.float().cpu() - rne).abs() <= tol).all()), f"P={P}: bf16 output off by more than one ulp"
        assert float((ob.float().cpu() == rne).float().mean()) >= 0.99


def test_boundary_sizes(gpu):
    ma = hip_attend.HipAttend()
    K4, V4, q5 = make(gpu, C=600)
    for S in (1, 5, 31, 32, 33, 255, 257, 600):
        rows3 = torch.stack([torch.randperm(600, generator=torch.Generator().manual_seed(S + g))[:S] for g in range(8)])[None]
        K, V, q, rows = hip_attend.model_views(K4, V4, q5, rows3.to(gpu))
        ref = ref_of(q5, K4, V4, rows3)[0]
        for P in PARTS:
            out = ma(K, V, q, rows, partitions=P)
            torch.cuda.synchronize()
            assert bool(torch.isfinite(out).all()), f"S={S} P={P}: non-finite (empty partition handling)"
            check(out, ref, f"S={S} P={P}")


def test_poisoned_unselected_rows_never_change_the_output(gpu):
    ma = hip_attend.HipAttend()
    K4, V4, q5 = make(gpu, C=2304)
    rows3, _ = row_list(8, 2304, 2176 + 65, 1 / 8)
    K, V, q, rows = hip_attend.model_views(K4, V4, q5, rows3.to(gpu))
    Kp, Vp = K4.clone(), V4.clone()
    for g in range(8):
        keep = torch.zeros(2304, dtype=torch.bool)
        keep[rows3[0, g]] = True
        Kp[0, g, ~keep.to(gpu)] = float("nan")
        Vp[0, g, ~keep.to(gpu)] = float("nan")
    for P in PARTS:
        clean = ma(K, V, q, rows, partitions=P)
        poisoned = ma(Kp[0], Vp[0], q, rows, partitions=P)
        torch.cuda.synchronize()
        assert bool(torch.isfinite(poisoned).all()), f"P={P}: an unselected row was read"
        assert torch.equal(poisoned, clean), f"P={P}: poison changed the output"


def test_rows_are_original_positions_and_order_does_not_matter(gpu):
    ma = hip_attend.HipAttend()
    K4, V4, q5 = make(gpu, C=1024)
    rows3, _ = row_list(8, 1024, 1000, 1 / 8)
    perm = torch.stack([torch.randperm(rows3.shape[-1], generator=torch.Generator().manual_seed(g)) for g in range(8)])
    shuffled = torch.stack([rows3[0, g][perm[g]] for g in range(8)])[None]
    K, V, q, rows = hip_attend.model_views(K4, V4, q5, rows3.to(gpu))
    _, _, _, rows_sh = hip_attend.model_views(K4, V4, q5, shuffled.to(gpu))
    a = ma(K, V, q, rows, partitions=4)
    b = ma(K, V, q, rows_sh, partitions=4)
    two = torch.tensor([2, 9]).view(1, 1, 2).expand(1, 8, 2).contiguous()
    _, _, _, r2 = hip_attend.model_views(K4, V4, q5, two.to(gpu))
    out2 = ma(K, V, q, r2, partitions=1)
    torch.cuda.synchronize()
    assert float((a - b).abs().max()) <= TOL["out_atol"], "row order changed the result beyond rounding"
    check(out2, ref_of(q5, K4, V4, two)[0], "positions 2 and 9")
    wrong = ref_of(q5, K4, V4, torch.tensor([0, 1]).view(1, 1, 2).expand(1, 8, 2).contiguous())[0]
    assert float(np.abs(f64(out2) - wrong).max()) > 1e-2, "rows were renumbered"
    assert float((a[:, 0] - a[:, 1]).abs().max()) > 1e-2, "the heads of a group must not share the answer"


def test_interleaved_kv_layout_diagnostic_matches(gpu):
    ma = hip_attend.HipAttend()
    K4, V4, q5 = make(gpu, C=2304)
    rows3, _ = row_list(8, 2304, 2176 + 65, 1 / 8)
    K, V, q, rows = hip_attend.model_views(K4, V4, q5, rows3.to(gpu))
    kv = torch.stack([K, V], dim=2).contiguous()
    ref = ref_of(q5, K4, V4, rows3)[0]
    for P in (1, 8):
        a = ma(K, V, q, rows, partitions=P)
        b = ma(None, None, q, rows, partitions=P, kv_interleaved=kv)
        torch.cuda.synchronize()
        check(b, ref, f"P={P} interleaved")
        assert float((a - b).abs().max()) <= 1e-6
    with pytest.raises(ValueError):
        ma(None, None, q, rows, partitions=1, kv_interleaved=kv.view(8, 2304, 256))


def test_validation(gpu):
    ma = hip_attend.HipAttend()
    K4, V4, q5 = make(gpu, C=600)
    rows3, _ = row_list(8, 600, 584, 1 / 8)
    K, V, q, rows = hip_attend.model_views(K4, V4, q5, rows3.to(gpu))
    with pytest.raises(ValueError):
        ma(K, V, q, rows3[0].to(gpu), partitions=4)                      # int64 rows
    with pytest.raises(ValueError):
        ma(K.float(), V, q, rows, partitions=4)
    with pytest.raises(ValueError):
        ma(K, V, q, rows, partitions=0)
    with pytest.raises(ValueError):
        ma(K[:, :, :64].contiguous(), V[:, :, :64].contiguous(), q[:, :, :64].contiguous(), rows, partitions=1)
    with pytest.raises(ValueError):
        hip_attend.model_views(torch.cat([K4, K4]), V4, q5, rows3.to(gpu))


@pytest.mark.parametrize("h", [1, 3, 4, 5, 8])
def test_head_counts(gpu, h):
    K4, V4, q5 = make(gpu, h=h, C=1500, seed=h, B=2)
    rows3, _ = row_list(8, 1500, 1400, 1 / 8, B=2)
    out = hip_attend.attend(q5[:, :, :, 0].contiguous(), K4, V4, rows3.to(torch.int32).to(gpu), out_dtype=torch.float32)
    torch.cuda.synchronize()
    check(out, ref_of(q5, K4, V4, rows3), f"h={h}")


@pytest.mark.parametrize("k", [64, 256, 1024, 2048])
def test_c3_shapes_sorted_and_unsorted(gpu, k):
    """Config 3: L = 32K, 16q/8kv, rows = 4 sinks + 128 most recent + k uniform picks, B in {1, 16} (B=16: k=1024)."""
    B = 16 if k == 1024 else 1
    L = C = 32768
    gen = torch.Generator().manual_seed(k)
    K4 = torch.randn(B, 8, C, 128, generator=gen).to(torch.bfloat16).to(gpu)
    V4 = torch.randn(B, 8, C, 128, generator=gen).to(torch.bfloat16).to(gpu)
    q = torch.randn(B, 8, 2, 128, generator=gen).to(torch.bfloat16).to(gpu)
    rows = []
    for _ in range(B * 8):
        picks = 4 + torch.randperm(L - 132, generator=gen)[:k]
        rows.append(torch.cat([torch.arange(4), torch.arange(L - 128, L), picks]))
    rows = torch.stack(rows).view(B, 8, -1)
    qn, Kn, Vn = f64(q), f64(K4), f64(V4)
    ref = exact.subset_attention(qn, Kn, Vn, rows.numpy())
    for rr in (rows, rows.sort(-1).values):
        out = hip_attend.attend(q, K4, V4, rr.to(torch.int32).to(gpu), out_dtype=torch.float32)
        torch.cuda.synchronize()
        check(out, ref, f"k={k}")
    dense = hip_attend.dense_decode(q, K4, V4, L, out_dtype=torch.float32)
    torch.cuda.synchronize()
    check(dense, exact.dense_attention(qn[:1], Kn[:1], Vn[:1], L) if B == 1 else exact.dense_attention(qn, Kn, Vn, L),
          "dense 32K")


@pytest.mark.parametrize("B,h,L,C", [(1, 2, 1, 8), (1, 2, 37, 37), (2, 4, 2048, 2100), (1, 8, 5000, 5000),
                                     (3, 1, 777, 800)])
def test_dense_decode_matches_oracle(gpu, B, h, L, C):
    K4, V4, q5 = make(gpu, h=h, C=C, seed=L, B=B)
    K4[:, :, L:] = float("nan")                                       # unwritten slots must never be read
    V4[:, :, L:] = float("nan")
    q = q5[:, :, :, 0].contiguous()
    ref = exact.dense_attention(f64(q), f64(K4), f64(V4), L)
    for P in (None, 1, 3, 16):
        out = hip_attend.dense_decode(q, K4, V4, L, partitions=P, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert bool(torch.isfinite(out).all())
        check(out, ref, f"dense L={L} P={P}")
    out5 = full_attention(q5, K4, V4, valid_length=L)
    torch.cuda.synchronize()
    assert out5.shape == q5.shape and out5.dtype == torch.bfloat16
    assert float(np.abs(f64(out5)[:, :, :, 0] - ref).max()) <= 2e-2


def test_full_attention_contract(gpu):
    K4, V4, q5 = make(gpu, C=64)
    with pytest.raises(ValueError):
        full_attention(q5, K4, V4, valid_length=200)
    with pytest.raises(ValueError):
        full_attention(q5, K4, V4, backend="flash")
    with pytest.raises(ValueError):
        full_attention(torch.cat([q5, q5], dim=3), K4, V4, valid_length=64, query_positions=[10])
    with pytest.raises(ValueError):
        full_attention(q5, K4, V4, valid_length=64, query_positions=[-1])
    # several queries (a prefill chunk): the reference's legality rule, key j legal iff j <= position and j < L
    q4 = torch.cat([q5, q5.flip(2), q5 * 0.5, -q5], dim=3)
    for L, qp in ((64, None), (50, [0, 17, 49, 60]), (64, [63, 2, 31, 31])):
        out = full_attention(q4, K4, V4, valid_length=L, query_positions=qp)
        torch.cuda.synchronize()
        want = exact.causal_attention(f64(q4), f64(K4), f64(V4), L, qp)
        assert float(np.abs(f64(out) - want).max()) <= 2e-2, f"L={L} positions={qp}"
    # one query before the last legal position reads only up to itself
    out = full_attention(q5, K4, V4, valid_length=64, query_positions=[10])
    torch.cuda.synchronize()
    assert float(np.abs(f64(out) - exact.causal_attention(f64(q5), f64(K4), f64(V4), 64, [10])).max()) <= 2e-2
    # a single query over the whole history: no square causal mask (test_attention_contracts.py:211-228)
    L = 37
    out = full_attention(q5, K4, V4, valid_length=L)
    torch.cuda.synchronize()
    q = f64(q5)[:, :, :, 0]
    s = np.einsum("bgid,bgcd->bgic", q, f64(K4)[:, :, :L]) / math.sqrt(128)
    p = np.exp(s - s.max(-1, keepdims=True))
    brute = np.einsum("bgic,bgcd->bgid", p / p.sum(-1, keepdims=True), f64(V4)[:, :, :L])
    assert float(np.abs(f64(out)[:, :, :, 0] - brute).max()) <= 2e-2


@pytest.mark.parametrize("h,T,masked", [(2, 1, False), (2, 3, True), (4, 2, False), (8, 1, True)])
def test_subset_attention_on_the_attend_kernel(gpu, h, T, masked):
    """subset_attention (sparse.py:40-60) over an already gathered subset: the h*T query rows of a group share its S
    rows; padded slots (valid_mask False) are not read, even when they hold NaN."""
    from attention_lab.sparse import gather_rows, subset_attention
    B, G, C, S = 2, 4, 600, 77
    gen = torch.Generator().manual_seed(h * 10 + T)
    K4 = torch.randn(B, G, C, 128, generator=gen).to(torch.bfloat16).to(gpu)
    V4 = torch.randn(B, G, C, 128, generator=gen).to(torch.bfloat16).to(gpu)
    q = torch.randn(B, G, h, T, 128, generator=gen).to(torch.bfloat16).to(gpu)
    sel = torch.stack([torch.randperm(C, generator=gen)[:S] for _ in range(B * G)]).view(B, G, S).to(gpu)
    k_sub, v_sub = gather_rows(K4, sel), gather_rows(V4, sel)
    valid = None
    slots = np.broadcast_to(np.arange(S), (B, G, S)).copy()
    if masked:
        valid = torch.rand(B, G, S, generator=gen).to(gpu) > 0.3
        k_sub[~valid] = float("nan")
        v_sub[~valid] = float("nan")
        slots = np.where(valid.cpu().numpy(), slots, -1)
    out = subset_attention(q, k_sub, v_sub, valid)
    torch.cuda.synchronize()
    assert out.shape == (B, G, h, T, 128) and out.dtype == torch.bfloat16
    qf = f64(q).reshape(B, G, h * T, 128)
    want = exact.subset_attention(qf, f64(k_sub), f64(v_sub), slots).reshape(B, G, h, T, 128)
    d = np.abs(f64(out) - want)
    assert np.isfinite(d).all() and d.max() <= 2e-2 and d.mean() <= 2e-3
    with pytest.raises(ValueError):
        subset_attention(torch.zeros(B, G, 8, 2, 128, dtype=torch.bfloat16, device=gpu), k_sub, v_sub)   # h*T > 8


@pytest.mark.parametrize("page,P,B,h", [(16, 1, 2, 2), (16, 8, 1, 4), (1, 4, 1, 2), (256, 2, 3, 1), (64, 16, 2, 8)])
def test_paged_cache_reads_exactly_what_the_contiguous_cache_reads(gpu, page, P, B, h):
    """The paged layout: pools of pages in a random order, unused pages NaN-poisoned, a block table per sequence.
    Over the same row lists the paged read equals the contiguous one bit for bit (same arithmetic, other addresses) and
    the float64 oracle within the bf16 bar; positions on an unmapped page (-1) are skipped."""
    G, C, L = 8, 2300, 2200
    K4, V4, q5 = make(gpu, G=G, h=h, C=C, seed=page + P, B=B)
    q = q5[:, :, :, 0].contiguous()
    rows = row_list(G, C, L, 1 / 16, seed=page, B=B)[0].to(torch.int32).to(gpu).contiguous()
    gen = torch.Generator().manual_seed(page)
    kp, vp, bt = hip_attend.page_cache(K4, V4, page, spare_pages=5, generator=gen)
    flat = hip_attend.attend(q, K4, V4, rows, partitions=P, out_dtype=torch.float32)
    paged = hip_attend.attend_paged(q, kp, vp, bt, rows, partitions=P, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(paged, flat), "paged and contiguous reads differ"
    ref = exact.subset_attention(f64(q), f64(K4), f64(V4), rows.cpu().numpy())
    assert np.abs(paged.double().cpu().numpy() - ref).max() <= TOL["out_atol"]
    # unmapped pages: drop the last logical page of every sequence from the table; its listed positions are skipped
    bt2 = bt.clone()
    last = (L - 1) // page
    bt2[:, last] = -1
    dropped = torch.where(rows // page == last, torch.full_like(rows, -1), rows)
    got = hip_attend.attend_paged(q, kp, vp, bt2, rows, partitions=P, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref2 = exact.subset_attention(f64(q), f64(K4), f64(V4), dropped.cpu().numpy())
    assert torch.isfinite(got).all() and np.abs(got.double().cpu().numpy() - ref2).max() <= TOL["out_atol"]


@pytest.mark.parametrize("page,C,L,listed", [(1, 5000, 4900, True), (2, 12000, 11000, False), (4, 12000, 11000, False),
                                           (8, 40000, 33000, True)])
def test_paged_long_block_tables_and_several_chunks(gpu, page, C, L, listed):
    """Block tables of up to 40000 / 8 = 5000 pages (page size 1 included) and the dense read of S > 4096 positions
    (several chunks of staged positions, each translated after its own barrier) agree bit for bit with the contiguous
    read."""
    G, B, h = 8, 1, 2
    K4, V4, q5 = make(gpu, G=G, h=h, C=C, seed=page + C, B=B)
    q = q5[:, :, :, 0].contiguous()
    kp, vp, bt = hip_attend.page_cache(K4, V4, page, spare_pages=3, generator=torch.Generator().manual_seed(C))
    if listed:
        rows = row_list(G, C, L, 1 / 16, seed=page, B=B)[0].to(torch.int32).to(gpu).contiguous()
        flat = hip_attend.attend(q, K4, V4, rows, partitions=4, out_dtype=torch.float32)
        got = hip_attend.attend_paged(q, kp, vp, bt, rows, partitions=4, out_dtype=torch.float32)
    else:
        rows_all = torch.arange(L, dtype=torch.int32, device=gpu).expand(B, G, L).contiguous()
        flat = hip_attend.attend(q, K4, V4, rows_all, partitions=2, out_dtype=torch.float32)
        got = hip_attend.attend_paged(q, kp, vp, bt, None, length=L, partitions=2, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(got, flat), "paged and contiguous reads differ"


@pytest.mark.parametrize("page,L", [(16, 2048), (128, 1000)])
def test_dense_read_of_a_paged_cache(gpu, page, L):
    """rows=None reads positions [0, L) of each sequence through its block table: the dense control over pages."""
    G, C, B, h = 8, 2048, 2, 2
    K4, V4, q5 = make(gpu, G=G, h=h, C=C, seed=L, B=B)
    q = q5[:, :, :, 0].contiguous()
    kp, vp, bt = hip_attend.page_cache(K4, V4, page, generator=torch.Generator().manual_seed(L))
    got = hip_attend.attend_paged(q, kp, vp, bt, None, length=L, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = exact.dense_attention(f64(q), f64(K4), f64(V4), L)
    assert np.abs(got.double().cpu().numpy() - ref).max() <= TOL["out_atol"]
