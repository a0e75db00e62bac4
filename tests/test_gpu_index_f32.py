"""Float32 index tables on the GPU: the trained bank's dtype (trained.py:11-18, 78-81) through the fp32 score, z
column, query projection, bulk build and the fused decode step, against the float64 oracle.

Bars, written here: scores and u within 1e-5 of the oracle on the same fp32 inputs (the north_star asks 1e-3
relative); the z column and the bulk build, sums of d fp32 products stored unrounded, within 128 * 2^-24 of the exact value
relative to the sum of |terms| (the error bound of any summation order of d = 128 fp32 terms; a dropped or doubled
term breaks it); row lists bit-exact against the oracle's top-k on the kernel's own fp32 scores;
attention output within the bf16 bar (max |d| <= 2e-2, mean |d| <= 2e-3).
"""
from __future__ import annotations

import hashlib
import json

import numpy as np
import pytest
import torch

from attention_lab import hip_score
from attention_lab.decode import prepare_request, sparse_decode_step_kernel
from attention_lab.indexer import GroupedIndexer, project_keys, project_queries
from oracle import bf16, exact, rules

pytestmark = pytest.mark.gpu
f64 = bf16.values
SCORE_ATOL = 1e-5
SUM_REL = 128 * 2.0 ** -24
BF16_MAX, BF16_MEAN = 2e-2, 2e-3


def a64(t):
    return t.detach().double().cpu().numpy()


def check_sum(got, exact_value, abs_terms, what):
    err = np.abs(a64(got) - exact_value)
    bound = SUM_REL * abs_terms + 1e-30
    assert np.all(err <= bound), f"{what}: worst err/bound {float((err / bound).max()):.2f}"


def setup(gpu, B, G, h, C, seed, r=32):
    gen = torch.Generator().manual_seed(seed)
    zT = torch.randn(B, G, r, C, generator=gen).to(gpu)
    q_pre = torch.randn(B, G, h, 1, 128, generator=gen).to(gpu)
    k_pre_new = torch.randn(B, G, 1, 128, generator=gen).to(gpu)
    idx = GroupedIndexer(G, h, 128, r, device=gpu, dtype=torch.float32, seed=seed)
    return zT, q_pre, k_pre_new, idx


@pytest.mark.parametrize("B,h,C,L", [(3, 2, 1024 + 64, 1024), (2, 4, 1001, 999), (1, 1, 4099, 4099),
                                     (16, 4, 32768, 32768)])
def test_score_u_and_z_column(gpu, B, h, C, L):
    """Aligned tables (16-byte loads) and C % 4 != 0 (4-byte loads), candidate ranges with ragged ends."""
    G = 8
    zT, q_pre, k_pre_new, idx = setup(gpu, B, G, h, C, seed=C + B)
    lo, hi, wc = 4, L - 64, L - 1
    q_cat = q_pre.reshape(B, G, h * 128).contiguous()
    k_new = k_pre_new.reshape(B, G, 128).contiguous()
    zw = zT.clone()
    u_out = torch.empty(B, G, 32, dtype=torch.float32, device=gpu)
    s = hip_score.score_grouped(zw, lo, hi, wk=idx.wk, q_cat=q_cat, wq_t=idx.wq_t_scaled, k_new=k_new, write_col=wc,
                                u_out=u_out)
    torch.cuda.synchronize()
    u = exact.grouped_u(a64(q_cat), a64(idx.wq_t_scaled))
    assert np.abs(a64(u_out) - u).max() <= SCORE_ATOL
    assert np.abs(a64(s) - exact.grouped_scores(u, a64(zT), lo, hi)).max() <= SCORE_ATOL
    z, _ = exact.z_column(a64(k_new), a64(idx.wk))
    terms = np.einsum("gjd,bgd->bgj", np.abs(a64(idx.wk)), np.abs(a64(k_new)))
    check_sum(zw[..., wc], z, terms, "z column")
    mask = torch.ones(C, dtype=torch.bool, device=gpu)
    mask[wc] = False
    assert torch.equal(zw[..., mask], zT[..., mask]), "the score wrote outside the z column"
    s2 = hip_score.score_grouped(zT, lo, hi, u=u_out)       # the scan from a given u is the same kernel
    torch.cuda.synchronize()
    assert torch.equal(s2, s)


def test_project_queries_and_keys(gpu):
    B, G, h, C, d = 2, 8, 2, 333, 128
    gen = torch.Generator().manual_seed(4)
    q_pre = torch.randn(B, G, h, 1, d, generator=gen).to(gpu)
    idx = GroupedIndexer(G, h, d, 32, device=gpu, dtype=torch.float32, seed=4)
    u = project_queries(q_pre, idx.wq_t_scaled)
    torch.cuda.synchronize()
    ref = exact.grouped_u(a64(q_pre).reshape(B, G, h * d), a64(idx.wq_t_scaled))
    assert np.abs(a64(u).reshape(B, G, 32) - ref).max() <= SCORE_ATOL
    # strided keys, as the wrapper hands them over ([B, T, G, d] transposed to [B, G, T, d]; batch 1 keeps the
    # strided form, a batch of two is made contiguous first)
    B = 1
    k_rows = torch.randn(B, C, G, d, generator=gen).to(gpu)
    k_pre = k_rows.transpose(1, 2)
    table = torch.full((B, G, 32, C + 7), float("nan"), device=gpu)
    bounds = [0, 1, 64, 200, C]
    for a, b in zip(bounds, bounds[1:]):
        project_keys(k_pre[:, :, a:b], idx.wk, out=table, col0=a)
    one = idx.keys(k_pre)
    torch.cuda.synchronize()
    assert one.dtype == torch.float32 and tuple(one.shape) == (B, G, 32, C)
    assert torch.equal(table[..., :C], one), "chunked build differs from the one-shot build"
    assert bool(torch.isnan(table[..., C:]).all()), "columns past the last chunk were written"
    want = exact.project_keys(a64(k_pre), a64(idx.wk))
    terms = exact.project_keys(np.abs(a64(k_pre)), np.abs(a64(idx.wk)))
    check_sum(one, want, terms, "bulk build")


@pytest.mark.parametrize("d,r,C", [(128, 16, 704), (128, 20, 702), (64, 32, 702), (96, 8, 705), (40, 32, 704)])
def test_project_keys_shapes(gpu, d, r, C):
    """Matrix-core build (d a multiple of 16: one or two 16-row tiles, the compile-time loop at d = 128, the runtime
    loop elsewhere) and the scalar build (d = 40): columns that are not 4-aligned (4-byte stores after the staged
    tile), chunk ends inside a 256-position workgroup, every column within the sum bound of the exact value."""
    B, G, T = 2, 3, 700
    gen = torch.Generator().manual_seed(d + r)
    k_pre = torch.randn(B, G, C, d, generator=gen).to(gpu)
    wk = (0.02 * torch.randn(G, r, d, generator=gen)).to(gpu)
    table = torch.full((B, G, r, C), float("nan"), device=gpu)
    bounds = [0, 5, 333, T]
    for a, b in zip(bounds, bounds[1:]):
        project_keys(k_pre[:, :, a:b], wk, out=table, col0=a)
    torch.cuda.synchronize()
    want = exact.project_keys(a64(k_pre[:, :, :T]), a64(wk))
    terms = exact.project_keys(np.abs(a64(k_pre[:, :, :T])), np.abs(a64(wk)))
    check_sum(table[..., :T], want, terms, f"bulk build d={d} r={r}")
    assert bool(torch.isnan(table[..., T:]).all()), "columns past the last chunk were written"


def test_project_keys_validation(gpu):
    idx = GroupedIndexer(2, 2, 128, 32, device=gpu, dtype=torch.float32, seed=1)
    k = torch.randn(1, 2, 10, 128, device=gpu)
    with pytest.raises(ValueError):
        project_keys(k.to(torch.bfloat16), idx.wk)                       # mixed dtypes
    with pytest.raises(ValueError):
        project_keys(k, idx.wk, out=torch.empty(1, 2, 32, 10, dtype=torch.bfloat16, device=gpu))


@pytest.mark.parametrize("B,h,C,L,rho,canonical", [
    (1, 2, 2048 + 64, 2048, 1 / 32, True),
    (2, 4, 3001, 2900, 1 / 8, False),
    (3, 1, 1000, 1000, 1 / 32, True),
    (1, 2, 200, 128, 1 / 8, False),
])
def test_step_matches_oracle(gpu, B, h, C, L, rho, canonical):
    G = 8
    zT, q_pre, k_pre_new, idx = setup(gpu, B, G, h, C, seed=L + C)
    gen = torch.Generator().manual_seed(L)
    K = torch.randn(B, G, C, 128, generator=gen).to(torch.bfloat16).to(gpu)
    V = torch.randn(B, G, C, 128, generator=gen).to(torch.bfloat16).to(gpu)
    q = torch.randn(B, G, h, 1, 128, generator=gen).to(torch.bfloat16).to(gpu)
    before = zT.clone()
    req = prepare_request(B, G, C, valid_length=L, query_position=L - 1, rho=rho, device=gpu)
    out, rows = sparse_decode_step_kernel(q, q_pre, K, V, zT, idx.wq_t_scaled, idx.wk, req.fixed_rows, req.off_lo,
                                          req.layout.candidate_lo, req.layout.candidate_hi, req.k, req.selected_count,
                                          k_pre_new=k_pre_new, write_col=req.write_col, return_rows=True,
                                          canonical_order=canonical)
    torch.cuda.synchronize()
    lo, hi, k, S = rules.step(L, req.k0)
    pos = (rows.view(B, G, -1) - req.offsets).cpu().numpy()
    assert pos.shape == (B, G, S)
    z, _ = exact.z_column(a64(k_pre_new).reshape(B, G, 128), a64(idx.wk))
    terms = np.einsum("gjd,bgd->bgj", np.abs(a64(idx.wk)), np.abs(a64(k_pre_new).reshape(B, G, 128)))
    check_sum(zT[..., L - 1], z, terms, "z column of the step")
    mask = torch.ones(C, dtype=torch.bool, device=gpu)
    mask[L - 1] = False
    assert torch.equal(zT[..., mask], before[..., mask])
    # the kernel's own scores (same prologue and scan), then the oracle's selection on them
    u_out = torch.empty(B, G, 32, dtype=torch.float32, device=gpu)
    s = hip_score.score_grouped(zT, lo, hi, q_cat=q_pre.reshape(B, G, h * 128).contiguous(), wq_t=idx.wq_t_scaled,
                                u_out=u_out)
    torch.cuda.synchronize()
    u = exact.grouped_u(a64(q_pre).reshape(B, G, h * 128), a64(idx.wq_t_scaled))
    assert np.abs(a64(s) - exact.grouped_scores(u, a64(zT), lo, hi)).max() <= SCORE_ATOL
    want = exact.select_rows(s.cpu().numpy(), lo, hi, L, k, order="position" if canonical else "score")
    assert np.array_equal(pos, want), "row list differs from the oracle"
    ref = exact.subset_attention(f64(q)[:, :, :, 0], f64(K), f64(V), want)
    d = np.abs(f64(out).reshape(ref.shape) - ref)
    assert d.max() <= BF16_MAX and d.mean() <= BF16_MEAN, f"max {d.max():.3e} mean {d.mean():.3e}"


def _shape_table(zT, lo, hi, case):
    """Candidate columns [lo, hi) rearranged so the scores stress the list select (as for bf16 tables): one tile far
    above the rest (its list is cut and the tile read in full), every score equal (one first-digit bin holds the row),
    seven distinct values (ties at the threshold across every list). Scaling by powers of two is exact in fp32."""
    M = hi - lo
    if case == "skewed_tile":
        zT[..., lo + M // 5: lo + M // 5 + 700] *= 4
        zT[..., hi - 300: hi] *= 2
    elif case == "all_equal":
        zT[..., lo:hi] = zT[..., lo:lo + 1].expand(*zT.shape[:-1], M)
    else:
        src = lo + (torch.arange(M, device=zT.device) * 5) % 7
        zT[..., lo:hi] = zT[..., src]


@pytest.mark.parametrize("case", ["skewed_tile", "all_equal", "seven_values"])
@pytest.mark.parametrize("B,h,C,L,rho", [
    (2, 2, 8192 + 64, 8192, 1 / 8),       # one 512-column sub-tile per score workgroup, M < 8192
    (1, 2, 16384 + 64, 16384, 1 / 16),    # M > 8192: an all-equal row overflows the select's LDS candidates
    (16, 4, 16384, 16384, 1 / 32),        # two sub-tiles per score workgroup
])
def test_step_list_select_on_hard_distributions(gpu, case, B, h, C, L, rho):
    """The float32 one-launch score's key lists through the list select, in both row orders, bit-exact against the
    oracle's selection on the kernel's own scores."""
    G = 8
    zT, q_pre, k_pre_new, idx = setup(gpu, B, G, h, C, seed=L + B)
    gen = torch.Generator().manual_seed(C)
    K = torch.randn(B, G, C, 128, generator=gen).to(torch.bfloat16).to(gpu)
    V = torch.randn(B, G, C, 128, generator=gen).to(torch.bfloat16).to(gpu)
    q = torch.randn(B, G, h, 1, 128, generator=gen).to(torch.bfloat16).to(gpu)
    req = prepare_request(B, G, C, valid_length=L, query_position=L - 1, rho=rho, device=gpu)
    lo, hi = req.layout.candidate_lo, req.layout.candidate_hi
    _shape_table(zT, lo, hi, case)
    for canonical in (True, False):
        z = zT.clone()
        out, rows = sparse_decode_step_kernel(q, q_pre, K, V, z, idx.wq_t_scaled, idx.wk, req.fixed_rows, req.off_lo,
                                              lo, hi, req.k, req.selected_count, k_pre_new=k_pre_new,
                                              write_col=req.write_col, return_rows=True, canonical_order=canonical)
        u_out = torch.empty(B, G, 32, dtype=torch.float32, device=gpu)
        s = hip_score.score_grouped(z, lo, hi, q_cat=q_pre.reshape(B, G, h * 128).contiguous(), wq_t=idx.wq_t_scaled,
                                    u_out=u_out)
        torch.cuda.synchronize()
        pos = (rows.view(B, G, -1) - req.offsets).cpu().numpy()
        want = exact.select_rows(s.cpu().numpy(), lo, hi, L, req.k, order="position" if canonical else "score")
        assert np.array_equal(pos, want), f"{case} canonical={canonical}: row list differs from the oracle"
        if canonical:
            ref = exact.subset_attention(f64(q)[:, :, :, 0], f64(K), f64(V), want)
            d = np.abs(f64(out).reshape(ref.shape) - ref)
            assert d.max() <= BF16_MAX and d.mean() <= BF16_MEAN, f"{case}: max {d.max():.3e} mean {d.mean():.3e}"


def test_step_validation(gpu):
    zT, q_pre, k_pre_new, idx = setup(gpu, 1, 8, 2, 300, seed=1)
    K = torch.zeros(1, 8, 300, 128, dtype=torch.bfloat16, device=gpu)
    req = prepare_request(1, 8, 300, valid_length=256, query_position=255, rho=1 / 8, device=gpu)
    args = (req.fixed_rows, req.off_lo, req.layout.candidate_lo, req.layout.candidate_hi, req.k, req.selected_count)
    with pytest.raises(ValueError):   # an fp32 table with a bfloat16 query projection
        sparse_decode_step_kernel(q_pre.to(torch.bfloat16), q_pre.to(torch.bfloat16), K, K, zT, idx.wq_t_scaled,
                                  idx.wk, *args)
    with pytest.raises(ValueError):   # the index new key must match the table's dtype
        sparse_decode_step_kernel(q_pre.to(torch.bfloat16), q_pre, K, K, zT, idx.wq_t_scaled, idx.wk, *args,
                                  k_pre_new=k_pre_new.to(torch.bfloat16), write_col=req.write_col)


# ---------------------------------------------------------------------------------------------------------------------
# the trained-bank wrapper path (reference tests/test_trained_inference.py:33-52, 65-90)
# ---------------------------------------------------------------------------------------------------------------------
transformers = pytest.importorskip("transformers")
from attention_lab.qwen_wrap import (LabRunner, LabState, geometry_of, make_cache, tiny_qwen3,  # noqa: E402
                                     unwrap_model, wrap_model)
from attention_lab.trained import load_bank, make_trained_state  # noqa: E402


def bank_for(model, tmp_path, r=4):
    geo = geometry_of(model)
    entries = []
    for layer in range(geo.layers):
        idx = GroupedIndexer(geo.groups, geo.heads_per_group, geo.head_dim, r, seed=100 + layer)
        path = tmp_path / f"layer-{layer}.npz"
        np.savez(path, wq=idx.wq.numpy(), wk=idx.wk.numpy())
        sha = hashlib.sha256(path.read_bytes()).hexdigest()
        entries.append(dict(layer_index=layer, initial_file=path.name, final_file=path.name, initial_sha256=sha,
                            final_sha256=sha))
    meta = dict(model_id="tiny-test", revision="fixture", r=r, layers=entries)
    meta["bank_id"] = hashlib.sha256(json.dumps(meta, sort_keys=True).encode()).hexdigest()
    return load_bank(tmp_path, meta, geo, device=next(model.parameters()).device)


def tiny(gpu):
    return tiny_qwen3(seed=3, layers=2, hidden=256, heads=4, groups=2, head_dim=128, intermediate=256, vocab=256,
                      dtype=torch.bfloat16).to(gpu)


@pytest.mark.parametrize("active_layers", [{0}, None])
def test_trained_state_every_candidate_equals_full(gpu, tmp_path, active_layers):
    """k0 = capacity selects every candidate: the sparse read over the fp32 index equals the full read (the
    reference's bf16 contract tolerance: the sparse attend and the dense decode kernels sum in different orders), and
    the fp32 table is finite over every written position, inactive layers included."""
    model = tiny(gpu)
    holder = wrap_model(model)
    bank = bank_for(model, tmp_path)
    with torch.inference_mode():
        st = make_trained_state(model, 96, bank, sparse_layers=active_layers)
        st.record_selection = True
        for z in st.cache.z:
            z.fill_(float("nan"))
        full = LabState(make_cache(model, 96, with_index=False), mode="full")
        a, dd = LabRunner(model, holder, full), LabRunner(model, holder, st)
        prefix = torch.arange(1, 81, device=gpu).view(1, -1)
        a.prefill(prefix, 16)
        dd.prefill(prefix, 16)
        st.begin_request(0.125, k0=96)
        for token in (81, 82, 83):
            t = torch.tensor([[token]], device=gpu)
            want, got = a.step(t).float(), dd.step(t).float()
            diff = (got - want).abs()
            rel = float(diff.norm() / want.norm())
            assert float(diff.max()) <= 5e-2 and rel <= 2e-2, f"token {token}: max {float(diff.max()):.3e} rel {rel:.3e}"
        assert st.cache.k[0].dtype == torch.bfloat16 and st.cache.z[0].dtype == torch.float32
        assert all(bool(torch.isfinite(z[..., :st.cache.valid_length]).all()) for z in st.cache.z)
        if active_layers == {0}:
            assert st.last_rows[0] is not None and st.last_rows[1] is None
        else:
            assert all(x is not None for x in st.last_rows)
    unwrap_model(model)


def test_trained_index_cache_holds_wk_of_the_pre_rope_keys(gpu, tmp_path):
    model = tiny(gpu)
    holder = wrap_model(model)
    bank = bank_for(model, tmp_path)
    st = make_trained_state(model, 96, bank, sparse_layers={0})
    run = LabRunner(model, holder, st)
    captured = [[], []]
    hooks = []
    for layer, block in enumerate(model.model.layers):
        def record(module, args, output, l=layer):
            captured[l].append(output.detach().float().transpose(1, 2))
        hooks.append(block.self_attn.inner.k_norm.register_forward_hook(record))
    try:
        with torch.inference_mode():
            run.prefill(torch.arange(1, 81, device=gpu).view(1, -1), 16)
            st.begin_request(0.125)
            run.step(torch.tensor([[81]], device=gpu))
            run.step(torch.tensor([[82]], device=gpu))
    finally:
        for hk in hooks:
            hk.remove()
    for layer in range(2):
        keys = a64(torch.cat(captured[layer], dim=2)[0])                  # [G, 82, d]
        w = a64(bank.indexes[layer].wk)
        want = np.einsum("grd,gnd->grn", w, keys)
        terms = np.einsum("grd,gnd->grn", np.abs(w), np.abs(keys))
        check_sum(st.cache.z[layer][0, :, :, :82], want, terms, f"layer {layer} index cache")
    unwrap_model(model)


def test_parameter_mutation_rejects_before_cache_write(gpu, tmp_path):
    model = tiny(gpu)
    holder = wrap_model(model)
    bank = bank_for(model, tmp_path)
    st = make_trained_state(model, 96, bank)
    run = LabRunner(model, holder, st)
    with torch.inference_mode():
        run.prefill(torch.ones(1, 80, dtype=torch.long, device=gpu), 16)
    st.begin_request(0.125)
    length, writes = st.cache.valid_length, list(st.cache.writes)
    bank.indexes[0].wk.add_(0.01)
    with torch.inference_mode(), pytest.raises(RuntimeError, match="parameters changed"):
        run.step(torch.tensor([[2]], device=gpu))
    assert st.cache.valid_length == length and st.cache.writes == writes
    unwrap_model(model)


@pytest.mark.parametrize("B,h,C,L,rho,case", [(1, 2, 32768 + 64, 32768, 1 / 32, None),
                                              (2, 4, 8192 + 64, 8192, 1 / 8, "skewed_tile"),
                                              (1, 2, 16384 + 64, 16384, 1 / 16, "all_equal")])
def test_step_without_rows_equals_the_separate_stages(gpu, B, h, C, L, rho, case):
    """Over float32 tables too, a step that returns no row list selects inside the attend's workgroups: its output
    equals, bit for bit, the same step asking for its rows in position order (separate select and attend launches),
    incomplete lists recomputed from the float32 table included."""
    G = 8
    zT, q_pre, k_pre_new, idx = setup(gpu, B, G, h, C, seed=L + 7)
    gen = torch.Generator().manual_seed(C)
    K = torch.randn(B, G, C, 128, generator=gen).to(torch.bfloat16).to(gpu)
    V = torch.randn(B, G, C, 128, generator=gen).to(torch.bfloat16).to(gpu)
    q = torch.randn(B, G, h, 1, 128, generator=gen).to(torch.bfloat16).to(gpu)
    req = prepare_request(B, G, C, valid_length=L, query_position=L - 1, rho=rho, device=gpu)
    lo, hi = req.layout.candidate_lo, req.layout.candidate_hi
    if case:
        _shape_table(zT, lo, hi, case)
    outs = []
    for rows in (False, True):
        z = zT.clone()
        got = sparse_decode_step_kernel(q, q_pre, K, V, z, idx.wq_t_scaled, idx.wk, req.fixed_rows, req.off_lo, lo, hi,
                                        req.k, req.selected_count, k_pre_new=k_pre_new, write_col=req.write_col,
                                        return_rows=rows, canonical_order=True)
        torch.cuda.synchronize()
        outs.append(got[0] if rows else got)
    assert torch.equal(outs[0], outs[1])
