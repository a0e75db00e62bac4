"""Score kernels on the GPU against the oracle (contracts of the reference's tests/test_metal_score.py).

Preset tolerances (test_metal_score.py:27): fp32 scores vs the float64 oracle on the same bf16 inputs, max |d| <= 1e-5
and relative norm <= 1e-5 (north_star asks only 1e-3 relative); z column within one bf16 ulp (2^-8 relative) of the
PyTorch bf16 path and >= 90% bitwise equal to it; the RNE of the exact z bitwise in >= 99%.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from attention_lab import hip_score
from attention_lab.decode import prepare_request
from attention_lab.indexer import GroupedIndexer, project_keys
from oracle import bf16, exact

pytestmark = pytest.mark.gpu
TOL = {"scores_atol": 1e-5, "scores_rel_norm": 1e-5, "z_rel_ulp": 2.0 ** -8}
f64 = bf16.values


def make(dev, G=8, h=2, d=128, r=32, C=600, seed=0, B=1):
    gen = torch.Generator().manual_seed(seed)
    zT4 = torch.randn(B, G, r, C, generator=gen).to(torch.bfloat16)
    k_pre_new = torch.randn(B, G, 1, d, generator=gen).to(torch.bfloat16)
    q_pre = torch.randn(B, G, h, 1, d, generator=gen).to(torch.bfloat16)
    idx = GroupedIndexer(G, h, d, r, device=dev, dtype=torch.bfloat16, seed=seed)
    return zT4.to(dev), k_pre_new.to(dev), q_pre.to(dev), idx


def case(dev, C, L, seed=0):
    zT4, k_pre_new, q_pre, idx = make(dev, C=C, seed=seed)
    req = prepare_request(1, 8, C, valid_length=L, query_position=L - 1, rho=1 / 8, device=dev)
    return zT4, k_pre_new, q_pre, idx, req.layout.candidate_lo, req.layout.candidate_hi, req.write_col


def oracle_scores(zT, k_new, wk, q_cat, wq_t, lo, hi):
    u = exact.grouped_u(f64(q_cat), f64(wq_t))
    return exact.grouped_scores(u, f64(zT), lo, hi)


def same_sum(a, b, what):
    """Two fp32 evaluations of the same 32-term sums in different orders (one kernel sums j sequentially, another in
    four partial sums): equal up to fp32 rounding of the terms, 32 * 2^-24 relative to the largest score."""
    scale = max(1.0, float(a.abs().max()))
    diff = float((a - b).abs().max())
    assert diff <= 32 * 2.0 ** -24 * scale * 4, f"{what}: {diff:.3e} apart (scale {scale:.2e})"


def check_scores(got, ref, what):
    got = f64(got)
    diff = float(np.abs(got - ref).max())
    rel = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    assert diff <= TOL["scores_atol"], f"{what}: max abs diff {diff:.3e}"
    assert rel <= TOL["scores_rel_norm"], f"{what}: rel norm {rel:.3e}"
    return diff


@pytest.mark.parametrize("C,L", [(600, 584), (1024, 1000), (2304, 2176 + 65), (2304, 2176 + 67), (601, 585),
                                 (2301, 2176 + 65), (1020, 1000), (4096, 4000)])
def test_fused_matches_oracle_and_two_launch(gpu, C, L):
    # M = 512, 932, 2173, 2175, 517, 2173, 932, 3932: tails of every residue; C % 8 != 0 takes the 2-byte scan
    hs = hip_score.HipScore()
    zT4, k_pre_new, q_pre, idx, lo, hi, wc = case(gpu, C, L)
    zT, k_new, wk, q_cat, wq_t = hip_score.model_views(zT4, k_pre_new, q_pre, idx)
    ref = oracle_scores(zT, k_new, wk, q_cat, wq_t, lo, hi)
    outs = {}
    for version in (1, 2):
        s1 = hs.fused(zT.clone(), k_new, wk, q_cat, wq_t, lo, hi, wc, version=version)
        s2 = hs.two_launch(zT.clone(), k_new, wk, q_cat, wq_t, lo, hi, wc, version=version)
        torch.cuda.synchronize()
        assert tuple(s1.shape) == (8, hi - lo)
        check_scores(s1, ref, f"v{version} fused")
        check_scores(s2, ref, f"v{version} two-launch")
        same_sum(s2, s1, f"v{version} two-launch vs fused")
        outs[version] = s1.cpu()
    same_sum(outs[1], outs[2], "v1 vs v2")
    # the PyTorch bf16 path (project_queries / candidate_scores in bf16) must not be more accurate
    qc, wqt, z = (t.cpu() for t in (q_cat, wq_t, zT))
    u_bf = torch.matmul(qc.unsqueeze(1), wqt).squeeze(1)
    s_pt = torch.matmul(u_bf.unsqueeze(1), z[:, :, lo:hi].contiguous()).squeeze(1)
    pt_diff = float(np.abs(f64(s_pt) - ref).max())
    assert float(np.abs(f64(outs[2]) - ref).max()) <= pt_diff


def test_z_column_written_once_within_one_bf16_ulp(gpu):
    hs = hip_score.HipScore()
    zT4, k_pre_new, q_pre, idx, lo, hi, wc = case(gpu, 1024, 1000)
    zT, k_new, wk, q_cat, wq_t = hip_score.model_views(zT4, k_pre_new, q_pre, idx)
    before = zT.clone()
    hs.fused(zT, k_new, wk, q_cat, wq_t, lo, hi, wc)
    torch.cuda.synchronize()
    got = zT[:, :, wc].cpu()
    want = torch.matmul(wk.cpu(), k_new.cpu().unsqueeze(-1)).squeeze(-1)       # PyTorch bf16 project_keys
    tol = TOL["z_rel_ulp"] * want.float().abs() + 1e-6
    assert bool(((got.float() - want.float()).abs() <= tol).all()), "z column differs by more than one bf16 ulp"
    assert float((got == want).float().mean()) >= 0.9
    _, z_bits = exact.z_column(f64(k_new), f64(wk))
    assert np.mean(bf16.from_torch(got) == z_bits) >= 0.99, "z column is not the RNE of the exact value"
    mask = torch.ones(zT.shape[-1], dtype=torch.bool, device=gpu)
    mask[wc] = False
    assert torch.equal(zT[:, :, mask], before[:, :, mask]), "a column other than write_col was modified"


def test_columns_outside_the_scan_may_be_garbage(gpu):
    hs = hip_score.HipScore()
    for L in (1000, 999, 998, 997):   # M % 8 = 4, 3, 2, 1: the last aligned group crosses hi
        zT4, k_pre_new, q_pre, idx, lo, hi, wc = case(gpu, 1024, L)
        zT, k_new, wk, q_cat, wq_t = hip_score.model_views(zT4, k_pre_new, q_pre, idx)
        poisoned = zT.clone()
        poisoned[:, :, :lo] = float("nan")
        poisoned[:, :, hi:] = float("nan")
        for version in (1, 2):
            for form in ("fused", "two_launch"):   # two_launch with C % 8 == 0 scans with 16-byte, split-r loads
                run = getattr(hs, form)
                clean = run(zT.clone(), k_new, wk, q_cat, wq_t, lo, hi, wc, version=version)
                p = poisoned.clone()
                out = run(p, k_new, wk, q_cat, wq_t, lo, hi, wc, version=version)
                torch.cuda.synchronize()
                assert bool(torch.isfinite(out).all()), f"L={L} v{version} {form}: a column outside [lo, hi) leaked"
                assert torch.equal(out, clean), f"L={L} v{version} {form}: poison changed the scores"
                assert bool(torch.isfinite(p[:, :, wc].float()).all()), "write_col must hold the new z"


def test_empty_candidate_range_still_writes_z(gpu):
    hs = hip_score.HipScore()
    zT4, k_pre_new, q_pre, idx = make(gpu, C=64)
    zT, k_new, wk, q_cat, wq_t = hip_score.model_views(zT4, k_pre_new, q_pre, idx)
    zT[:, :, 40] = float("nan")
    s = hs.fused(zT, k_new, wk, q_cat, wq_t, 4, 4, 40)
    torch.cuda.synchronize()
    assert s.shape == (8, 0)
    assert bool(torch.isfinite(zT[:, :, 40].float()).all())


def test_validation(gpu):
    hs = hip_score.HipScore()
    zT4, k_pre_new, q_pre, idx, lo, hi, wc = case(gpu, 600, 584)
    zT, k_new, wk, q_cat, wq_t = hip_score.model_views(zT4, k_pre_new, q_pre, idx)
    with pytest.raises(ValueError):
        hs.fused(zT, k_new, wk, q_cat, wq_t, lo, hi, (lo + hi) // 2)
    with pytest.raises(ValueError):
        hs.fused(zT.float(), k_new, wk, q_cat, wq_t, lo, hi, wc)
    with pytest.raises(ValueError):
        hs.fused(zT.transpose(1, 2), k_new, wk, q_cat, wq_t, lo, hi, wc)
    with pytest.raises(ValueError):
        hip_score.model_views(torch.cat([zT4, zT4]), k_pre_new, q_pre, idx)
    with pytest.raises(ValueError):
        hs.fused(zT.cpu(), k_new.cpu(), wk.cpu(), q_cat.cpu(), wq_t.cpu(), lo, hi, wc)
    with pytest.raises(ValueError):
        hs.fused(zT, k_new, wk, q_cat, wq_t, lo, 601, wc)


@pytest.mark.parametrize("B,h,C,L", [(4, 2, 2048 + 64, 2048), (3, 4, 1000, 777), (16, 4, 32768, 32768)])
def test_batched_score_and_z(gpu, B, h, C, L):
    zT4, k_pre_new, q_pre, idx = make(gpu, B=B, h=h, C=C, seed=B)
    lo, hi = 4, L - 64
    wc = L - 1
    q_cat = q_pre.reshape(B, 8, h * 128).contiguous()
    k_new = k_pre_new.reshape(B, 8, 128).contiguous()
    u_out = torch.empty(B, 8, 32, dtype=torch.float32, device=gpu)
    zw = zT4.clone()
    s = hip_score.score_grouped(zw, lo, hi, wk=idx.wk, q_cat=q_cat, wq_t=idx.wq_t_scaled, k_new=k_new, write_col=wc,
                                u_out=u_out)
    torch.cuda.synchronize()
    u = exact.grouped_u(f64(q_cat), f64(idx.wq_t_scaled))
    assert np.abs(f64(u_out) - u).max() <= 1e-5
    check_scores(s, exact.grouped_scores(u, f64(zT4), lo, hi), f"B={B}")
    _, z_bits = exact.z_column(f64(k_new), f64(idx.wk))
    assert np.mean(bf16.from_torch(zw[..., wc]) == z_bits) >= 0.99
    # scan from a given u equals the fused scan
    s2 = hip_score.score_grouped(zT4, lo, hi, u=u_out)
    torch.cuda.synchronize()
    same_sum(s2, s, f"B={B} scan from u vs two-launch")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("nh,relu", [(1, False), (2, True), (4, True), (8, False), (3, True)])
def test_lightning_matches_oracle(gpu, dtype, nh, relu):
    B, KG, L = 2, 3, 5000
    gen = torch.Generator().manual_seed(nh)
    keys = (torch.randn(B, KG, L, 32, generator=gen) / 32 ** 0.5).to(dtype)
    q = torch.randn(B, KG, nh, 32, generator=gen)
    w = torch.rand(B, KG, nh, generator=gen)
    lo, hi = 4, L - 64
    s = hip_score.score_lightning(keys.to(gpu), q.to(gpu), w.to(gpu), lo, hi, relu=relu)
    torch.cuda.synchronize()
    ref = exact.lightning_scores(f64(keys), f64(q), f64(w), lo, hi, relu)
    assert np.abs(f64(s) - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("B,KG,L,ngroups", [(1, 8, 70000, 2), (2, 8, 90000, 5), (2, 8, 140000, 8)])
def test_lightning_long_rows_every_pipeline_depth(gpu, B, KG, L, ngroups):
    """Rows long enough for 2, 5 and 8 64-key groups per wave and tile (the kernel's three-group pipeline, whose group
    counts leave no load past a tile), the last tile of each row partial, lo > 0; against the float64 oracle."""
    nh = 4
    gen = torch.Generator().manual_seed(L)
    keys = (torch.randn(B, KG, L, 32, generator=gen) / 32 ** 0.5).to(torch.float16)
    q = torch.randn(B, KG, nh, 32, generator=gen)
    w = torch.rand(B, KG, nh, generator=gen)
    lo, hi = 68, L - 3
    per = (hi - lo) * B * KG // 262144   # the host's groups per tile: 8, 5, 2 or 1, the largest not above per
    assert (8 if per >= 8 else 5 if per >= 5 else 2 if per >= 2 else 1) == ngroups
    s = hip_score.score_lightning(keys.to(gpu), q.to(gpu), w.to(gpu), lo, hi, relu=True)
    torch.cuda.synchronize()
    ref = exact.lightning_scores(f64(keys), f64(q), f64(w), lo, hi, True)
    assert np.abs(f64(s) - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


def test_lightning_reduces_to_grouped_mode(gpu):
    """nh = 1, w = 1, identity activation, keys = zT transposed: the lightning kernel must equal the grouped scan."""
    B, G, C = 2, 8, 3000
    gen = torch.Generator().manual_seed(5)
    zT = torch.randn(B, G, 32, C, generator=gen).to(torch.bfloat16).to(gpu)
    u = torch.randn(B, G, 32, generator=gen).to(gpu)
    keys = zT.transpose(2, 3).contiguous()
    lo, hi = 4, C - 64
    grouped = hip_score.score_grouped(zT, lo, hi, u=u)
    light = hip_score.score_lightning(keys, u.view(B, G, 1, 32).contiguous(), torch.ones(B, G, 1, device=gpu), lo, hi,
                                      relu=False)
    torch.cuda.synchronize()
    assert float((grouped - light).abs().max()) <= 1e-5


def test_project_keys_and_chunked_build(gpu):
    B, G, C, d = 2, 8, 300, 128
    gen = torch.Generator().manual_seed(3)
    k_pre = torch.randn(B, G, C, d, generator=gen).to(torch.bfloat16).to(gpu)
    idx = GroupedIndexer(G, 2, d, 32, device=gpu, dtype=torch.bfloat16, seed=3)
    zT = idx.keys(k_pre)
    torch.cuda.synchronize()
    assert tuple(zT.shape) == (B, G, 32, C) and zT.is_contiguous()
    ref = exact.project_keys(f64(k_pre), f64(idx.wk))
    bits = bf16.from_f32(ref.astype(np.float32))
    assert np.mean(bf16.from_torch(zT) == bits) >= 0.99
    assert np.all(np.abs(f64(zT) - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-6)
    table = torch.full((B, G, 32, C + 16), float("nan"), dtype=torch.bfloat16, device=gpu)
    bounds = [0, 5, C // 2, C]
    for a, b in zip(bounds, bounds[1:]):
        project_keys(k_pre[:, :, a:b], idx.wk, out=table, col0=a)
    torch.cuda.synchronize()
    assert torch.equal(table[..., :C], zT), "chunked build differs from the one-shot build"
    assert bool(torch.isnan(table[..., C:].float()).all()), "columns past the chunk were written"


@pytest.mark.parametrize("d,r,C", [(128, 32, 704), (128, 20, 702), (64, 32, 702), (32, 8, 704), (40, 32, 704)])
def test_project_keys_shapes(gpu, d, r, C):
    """Matrix-core build (d a multiple of 32) and the LDS build (d = 40): every r, columns that are not 4-aligned
    (8-byte or 2-byte stores), chunk ends inside a 256-position workgroup, RNE of the exact value."""
    B, G, T = 2, 3, 700
    gen = torch.Generator().manual_seed(d + r)
    k_pre = torch.randn(B, G, C, d, generator=gen).to(torch.bfloat16).to(gpu)
    wk = (0.02 * torch.randn(G, r, d, generator=gen)).to(torch.bfloat16).to(gpu)
    ref = exact.project_keys(f64(k_pre[:, :, :T]), f64(wk))
    bits = bf16.from_f32(ref.astype(np.float32))
    table = torch.full((B, G, r, C), float("nan"), dtype=torch.bfloat16, device=gpu)
    bounds = [0, 5, 333, T]
    for a, b in zip(bounds, bounds[1:]):
        project_keys(k_pre[:, :, a:b], wk, out=table, col0=a)
    torch.cuda.synchronize()
    got = table[..., :T]
    assert np.mean(bf16.from_torch(got) == bits) >= 0.99
    assert np.all(np.abs(f64(got) - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-6)
    assert bool(torch.isnan(table[..., T:].float()).all()), "columns past the last chunk were written"
