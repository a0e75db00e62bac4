"""The whole sparse decode step (z column -> score -> top-k -> row list -> gather-free attend) against the oracle.

Bars: row lists bit-exact against the oracle's top-k on the kernel's own fp32 scores; scores within 1e-5 of the
float64 oracle; z column >= 99% bitwise equal to the RNE of the exact value; attention output within north_star's bf16
tolerance (max |d| <= 2e-2, mean |d| <= 2e-3) of the float64 subset attention over the same rows. Invariants from the
reference's contracts: NaN poison in unselected or unwritten rows is inert, every candidate selected (k = M) equals
the dense read, legal <= 68 degenerates to the dense read, rows are original positions.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from attention_lab import hip_attend, hip_score, hip_select
from attention_lab.decode import (dense_decode_step, gathered_decode_step_kernel, prepare_request,
                                  select_rows_kernel, sparse_decode_step, sparse_decode_step_kernel)
from attention_lab.indexer import GroupedIndexer
from oracle import bf16, exact, rules

pytestmark = pytest.mark.gpu
f64 = bf16.values
BF16_MAX, BF16_MEAN = 2e-2, 2e-3


def setup(gpu, B=1, G=8, h=2, C=2048 + 64, seed=0, r=32):
    gen = torch.Generator().manual_seed(seed)
    t = lambda *s: torch.randn(*s, generator=gen).to(torch.bfloat16).to(gpu)  # noqa: E731
    K, V = t(B, G, C, 128), t(B, G, C, 128)
    q, q_pre, k_pre_new = t(B, G, h, 1, 128), t(B, G, h, 1, 128), t(B, G, 1, 128)
    zT = t(B, G, r, C)
    idx = GroupedIndexer(G, h, 128, r, device=gpu, dtype=torch.bfloat16, seed=seed)
    return K, V, q, q_pre, k_pre_new, zT, idx


def run_step(gpu, K, V, q, q_pre, k_pre_new, zT, idx, L, rho, canonical, n0=None, workspace=None):
    B, G, C = K.shape[0], K.shape[1], K.shape[2]
    req = prepare_request(B, G, C, valid_length=L, query_position=L - 1, rho=rho, device=gpu, n0=n0)
    out, rows = sparse_decode_step_kernel(q, q_pre, K, V, zT, idx.wq_t_scaled, idx.wk, req.fixed_rows, req.off_lo,
                                          req.layout.candidate_lo, req.layout.candidate_hi, req.k, req.selected_count,
                                          k_pre_new=k_pre_new, write_col=req.write_col, return_rows=True,
                                          canonical_order=canonical, workspace=workspace)
    torch.cuda.synchronize()
    pos = (rows.view(B, G, -1) - req.offsets).cpu().numpy()
    return req, out, pos


def kernel_scores(zT, q_pre, idx, lo, hi):
    """Scores exactly as the fused step computes them: u by the prologue kernel, then the scan from u (the same fp32
    summation order, so the step's selection can be checked bit-exact against the oracle's on these scores)."""
    B, G, h, _, d = q_pre.shape
    u_out = torch.empty(B, G, idx.wq_t_scaled.shape[-1], dtype=torch.float32, device=zT.device)
    s = hip_score.score_grouped(zT, lo, hi, q_cat=q_pre.reshape(B, G, h * d).contiguous(), wq_t=idx.wq_t_scaled,
                                u_out=u_out)
    torch.cuda.synchronize()
    return s.cpu().numpy()


def check_out(out, ref, what):
    o = f64(out).reshape(ref.shape)
    d = np.abs(o - ref)
    assert d.max() <= BF16_MAX and d.mean() <= BF16_MEAN, f"{what}: max {d.max():.3e} mean {d.mean():.3e}"


@pytest.mark.parametrize("B,h,C,L,rho,canonical", [
    (1, 2, 2048 + 64, 2048, 1 / 32, True),      # config 1: k = 64, S = 132
    (1, 2, 2048 + 64, 2048, 1 / 32, False),
    (2, 4, 3000, 2900, 1 / 8, True),
    (1, 2, 300, 256, 1 / 8, False),             # (lo, hi, k) = (4, 192, 32)
    (1, 2, 200, 128, 1 / 8, True),              # (68, 16, 84)
    (3, 1, 1000, 1000, 1 / 32, False),
    (1, 2, 32768 + 64, 32768, 1 / 2, False),    # score order past the LDS sort: k = 16384 (radix pass)
    (1, 2, 32768 + 64, 32768, 0.3, False),      # k = 9830: past the LDS sort, inside the list select's k range
    (2, 2, 16384 + 64, 16384, 0.55, False),     # k = 8974 of M = 16316
    (1, 2, 32768, 32768, 1.0, False),           # every candidate, score order: k = M = 32700
])
def test_step_matches_oracle(gpu, B, h, C, L, rho, canonical):
    from attention_lab import _native as nat
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=B, h=h, C=C, seed=L)
    zT_before = zT.clone()
    ws = nat.Workspace()
    req, out, pos = run_step(gpu, K, V, q, q_pre, k_pre_new, zT, idx, L, rho, canonical, workspace=ws)
    torch.cuda.synchronize()
    assert int(ws.bytes(gpu, 0, "state").abs().sum()) == 0, "the step left its select state dirty"
    lo, hi, k, S = rules.step(L, req.k0)
    assert (req.layout.candidate_lo, req.layout.candidate_hi, req.k, req.selected_count) == (lo, hi, k, S)
    assert pos.shape == (B, 8, S)
    # z column written, nothing else
    z, z_bits = exact.z_column(f64(k_pre_new).reshape(B, 8, 128), f64(idx.wk))
    assert np.mean(bf16.from_torch(zT[..., L - 1]) == z_bits) >= 0.99
    mask = torch.ones(C, dtype=torch.bool, device=gpu)
    mask[L - 1] = False
    assert torch.equal(zT[..., mask], zT_before[..., mask])
    # scores within 1e-5 of the oracle; rows bit-exact against the oracle's selection on those scores
    s = kernel_scores(zT, q_pre, idx, lo, hi)
    u = exact.grouped_u(f64(q_pre).reshape(B, 8, h * 128), f64(idx.wq_t_scaled))
    assert np.abs(s - exact.grouped_scores(u, f64(zT), lo, hi)).max() <= 1e-5
    want = exact.select_rows(s, lo, hi, L, k, order="position" if canonical else "score")
    assert np.array_equal(pos, want), "row list differs from the oracle"
    ref = exact.subset_attention(f64(q)[:, :, :, 0], f64(K), f64(V), want)
    check_out(out, ref, "sparse step")


def test_every_candidate_selected_equals_dense(gpu):
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=2, C=1200, seed=9)
    L = 1100
    req, out, pos = run_step(gpu, K, V, q, q_pre, k_pre_new, zT, idx, L, 1.0, True)
    assert req.selected_count == L
    assert np.array_equal(pos, np.broadcast_to(np.arange(L), pos.shape))
    dense = dense_decode_step(q, K, V, L)
    torch.cuda.synchronize()
    assert float((out.float() - dense.float()).abs().max()) <= 1e-2
    check_out(out, exact.dense_attention(f64(q)[:, :, :, 0], f64(K), f64(V), L), "k = M vs dense")


@pytest.mark.parametrize("L,rho,k_expect,S_expect", [(60, 1 / 8, 0, 60), (128, 0.0, 0, 68), (40, 1.0, 0, 40)])
def test_short_history_and_zero_budget(gpu, L, rho, k_expect, S_expect):
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, C=256, seed=L)
    req, out, pos = run_step(gpu, K, V, q, q_pre, k_pre_new, zT, idx, L, rho, False)
    assert (req.k, req.selected_count) == (k_expect, S_expect)
    assert np.array_equal(pos[0, 0], np.array(rules.fixed_positions(L)))
    ref = exact.subset_attention(f64(q)[:, :, :, 0], f64(K), f64(V), pos)
    check_out(out, ref, "F only")
    _, z_bits = exact.z_column(f64(k_pre_new).reshape(1, 8, 128), f64(idx.wk))
    assert np.mean(bf16.from_torch(zT[..., L - 1]) == z_bits) >= 0.99


def test_k0_fixed_by_n0_then_clamped(gpu):
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, C=128, seed=1)
    req, out, pos = run_step(gpu, K, V, q, q_pre, k_pre_new, zT, idx, 100, 1 / 32, True, n0=8192)
    assert (req.k0, req.k, req.selected_count) == (256, 32, 100)
    assert np.array_equal(pos[0, 0], np.arange(100))


def test_poisoned_unselected_and_unwritten_rows_are_inert(gpu):
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, C=2304, seed=4)
    L = 2200
    zc = zT.clone()
    _, clean, pos = run_step(gpu, K, V, q, q_pre, k_pre_new, zc, idx, L, 1 / 16, True)
    Kp, Vp, zp = K.clone(), V.clone(), zT.clone()
    for g in range(8):
        keep = torch.zeros(2304, dtype=torch.bool)
        keep[torch.from_numpy(pos[0, g])] = True
        Kp[0, g, ~keep.to(gpu)] = float("nan")
        Vp[0, g, ~keep.to(gpu)] = float("nan")
    zp[..., L:] = float("nan")                                     # unwritten index columns
    zp[..., L - 1] = float("nan")                                  # the column the step writes
    _, poisoned, pos2 = run_step(gpu, Kp, Vp, q, q_pre, k_pre_new, zp, idx, L, 1 / 16, True)
    assert np.array_equal(pos, pos2)
    assert bool(torch.isfinite(poisoned.float()).all()), "D read a row it did not select"
    assert torch.equal(poisoned, clean)
    dense = dense_decode_step(q, Kp, Vp, L)
    torch.cuda.synchronize()
    assert not bool(torch.isfinite(dense.float()).all()), "the dense read must see the poison"


def test_reference_api_paths(gpu):
    """select_rows_kernel / gathered_decode_step_kernel / DecodeRequest / sparse_decode_step agree with the fused step."""
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=2, C=1100, seed=5)
    L = 1024
    req = prepare_request(2, 8, 1100, valid_length=L, query_position=L - 1, rho=1 / 8, device=gpu)
    z1 = zT.clone()
    out_a = sparse_decode_step(q, q_pre, K, V, z1, idx, req, k_pre_new=k_pre_new)
    u = idx.query(q_pre)
    rows = select_rows_kernel(u, z1, req.fixed_rows, req.off_lo, req.layout.candidate_lo, req.layout.candidate_hi, req.k)
    pos_sel = req.select_positions(u, z1)
    out_b = gathered_decode_step_kernel(q, K, V, rows, req.selected_count)
    # a step whose row list does not leave the call reads its rows in position order (the faster select): over the
    # same rows in that order the gathered read is the same bit for bit; over the score-ordered list only the
    # summation order differs, so at most one bf16 ulp
    by_pos = rows.view(2, 8, -1).sort(-1).values.reshape(-1)
    out_c = gathered_decode_step_kernel(q, K, V, by_pos, req.selected_count)
    torch.cuda.synchronize()
    assert torch.equal((rows.view(2, 8, -1) - req.offsets), pos_sel), "row ids and positions disagree"
    assert torch.equal(out_a, out_c)
    ulp = out_c.float().abs() * 2.0 ** -7 + 1e-6   # one bf16 ulp is at most 2^-7 of the value
    assert bool(((out_b.float() - out_a.float()).abs() <= ulp).all())
    lo, hi = req.layout.candidate_lo, req.layout.candidate_hi
    s = kernel_scores(z1, q_pre, idx, lo, hi)
    assert np.array_equal(pos_sel.cpu().numpy(), exact.select_rows(s, lo, hi, L, req.k, order="score"))
    top = pos_sel[..., req.layout.fixed_count:]
    assert bool(((top >= lo) & (top < hi)).all()), "chosen candidates must stay inside the candidate domain"


def test_full_size_32k_b16_properties(gpu):
    """C5 attention geometry at one layer: B=16, 32K, 8 KV groups, h=4, rho=1/32 -> k=1024, S=1092."""
    B, G, h, L = 16, 8, 4, 32768
    C = L
    dev = gpu
    torch.manual_seed(0)
    K = torch.randn(B, G, C, 128, device=dev, dtype=torch.bfloat16)
    V = torch.randn(B, G, C, 128, device=dev, dtype=torch.bfloat16)
    zT = torch.randn(B, G, 32, C, device=dev, dtype=torch.bfloat16)
    q = torch.randn(B, G, h, 1, 128, device=dev, dtype=torch.bfloat16)
    q_pre = torch.randn(B, G, h, 1, 128, device=dev, dtype=torch.bfloat16)
    k_pre_new = torch.randn(B, G, 1, 128, device=dev, dtype=torch.bfloat16)
    idx = GroupedIndexer(G, h, 128, 32, device=dev, dtype=torch.bfloat16, seed=0)
    req, out, pos = run_step(dev, K, V, q, q_pre, k_pre_new, zT, idx, L, 1 / 32, True)
    assert (req.k, req.selected_count) == (1024, 1092)
    assert np.all(np.diff(pos, axis=-1) > 0), "canonical rows must be strictly ascending (sorted, unique)"
    assert pos.min() >= 0 and pos.max() < L
    fixed = np.array(rules.fixed_positions(L))
    assert np.array_equal(pos[..., :4], np.broadcast_to(fixed[:4], (B, G, 4)))
    assert np.array_equal(pos[..., -64:], np.broadcast_to(fixed[4:], (B, G, 64)))
    lo, hi = req.layout.candidate_lo, req.layout.candidate_hi
    s = kernel_scores(zT, q_pre, idx, lo, hi)
    assert np.array_equal(pos, exact.select_rows(s, lo, hi, L, 1024, order="position"))
    ref = exact.subset_attention(f64(q)[:, :, :, 0], f64(K), f64(V), pos)
    check_out(out, ref, "32K B16")


def score_grid(B, G, lo, hi):
    """Workgroups of the one-launch score (8, 4 or 2 sub-tiles of 512 columns each, as many as leave 256 workgroups)."""
    span = ((hi + 7) & ~7) - (lo & ~7)
    blocks = B * G * ((span + 511) // 512)
    nsub = 8 if blocks >= 2048 else 4 if blocks >= 1024 else 2 if blocks >= 512 else 1
    return B * G * ((span + 512 * nsub - 1) // (512 * nsub))


@pytest.mark.parametrize("B,L,canonical", [(16, 16384, True), (8, 32768, False), (16, 32768, True), (4, 32768, True)])
def test_z_column_is_the_same_bits_whichever_kernel_writes_it(gpu, B, L, canonical):
    """The step's score kernel writes the new key's z column at the end of its tile-0 workgroups past one workgroup per
    CU, and ahead of the table (with u) in smaller grids. Either way the column is bit for bit the one
    attnlab_score_grouped writes on its own (write_z), at least 99% of it is the RNE of the exact value, no other column
    of zT changes, and the rows are bit-exact against the oracle."""
    G, h, C = 8, 2, L + 64
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=B, h=h, C=C, seed=B + L)
    z_step = zT.clone()
    req, out, pos = run_step(gpu, K, V, q, q_pre, k_pre_new, z_step, idx, L, 1 / 32, canonical)
    lo, hi = req.layout.candidate_lo, req.layout.candidate_hi
    assert (score_grid(B, G, lo, hi) > 256) == (B >= 8), "the cases cover both forms"
    z_score = zT.clone()
    hip_score.score_grouped(z_score, lo, hi, wk=idx.wk, q_cat=q_pre.reshape(B, G, h * 128).contiguous(),
                            wq_t=idx.wq_t_scaled, k_new=k_pre_new.reshape(B, G, 128).contiguous(), write_col=L - 1)
    torch.cuda.synchronize()
    assert torch.equal(z_step, z_score), "the step's z column differs from the score kernel's"
    _, z_bits = exact.z_column(f64(k_pre_new).reshape(B, G, 128), f64(idx.wk))
    assert np.mean(bf16.from_torch(z_step[..., L - 1]) == z_bits) >= 0.99
    mask = torch.ones(C, dtype=torch.bool, device=gpu)
    mask[L - 1] = False
    assert torch.equal(z_step[..., mask], zT[..., mask])
    want = exact.select_rows(kernel_scores(z_step, q_pre, idx, lo, hi), lo, hi, L, req.k,
                             order="position" if canonical else "score")
    assert np.array_equal(pos, want)


def test_graph_replay_matches_eager(gpu):
    """The launches of a step captured in a HIP graph: every replay equals the eager result."""
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=4, h=4, C=4096, seed=8)
    L = 4000
    req = prepare_request(4, 8, 4096, valid_length=L, query_position=L - 1, rho=1 / 32, device=gpu)
    args = (q, q_pre, K, V, zT, idx.wq_t_scaled, idx.wk, req.fixed_rows, req.off_lo, req.layout.candidate_lo,
            req.layout.candidate_hi, req.k, req.selected_count)
    kw = dict(k_pre_new=k_pre_new, write_col=req.write_col, canonical_order=True)
    eager = sparse_decode_step_kernel(*args, **kw).clone()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        sparse_decode_step_kernel(*args, **kw)                      # warm the workspace on the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        captured = sparse_decode_step_kernel(*args, **kw)
    for _ in range(3):
        captured.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager)
        dense_decode_step(q, K, V, L)                               # eager work between replays
        torch.cuda.synchronize()


def test_graph_replay_survives_workspace_growth(gpu):
    """A graph captured on a workspace, then a larger eager call that grows it: the retired buffers stay alive, so every
    replay still equals the eager result of the captured shape, and the larger call is bit-exact against the oracle."""
    from attention_lab import _native as nat
    ws = nat.Workspace()
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=2, h=2, C=2048 + 64, seed=21)
    L = 2048
    req = prepare_request(2, 8, 2048 + 64, valid_length=L, query_position=L - 1, rho=1 / 32, device=gpu)
    args = (q, q_pre, K, V, zT, idx.wq_t_scaled, idx.wk, req.fixed_rows, req.off_lo, req.layout.candidate_lo,
            req.layout.candidate_hi, req.k, req.selected_count)
    kw = dict(canonical_order=True, workspace=ws)
    eager = sparse_decode_step_kernel(*args, **kw).clone()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        sparse_decode_step_kernel(*args, **kw)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        captured = sparse_decode_step_kernel(*args, **kw)
    small = ws.bytes(gpu, 0, "step").numel()
    # a larger eager step (B=4, 8K context) grows the workspace; torch may hand the retired memory to no one else
    K2, V2, q2, q_pre2, k_new2, zT2, idx2 = setup(gpu, B=4, h=2, C=8192 + 64, seed=22)
    _, out2, pos2 = run_step(gpu, K2, V2, q2, q_pre2, k_new2, zT2, idx2, 8192, 1 / 16, True, workspace=ws)
    assert ws.bytes(gpu, 0, "step").numel() > small and ws.retired_bytes() >= small
    lo2, hi2 = 4, 8192 - 64
    s2 = kernel_scores(zT2, q_pre2, idx2, lo2, hi2)
    assert np.array_equal(pos2, exact.select_rows(s2, lo2, hi2, 8192, pos2.shape[-1] - 68, order="position"))
    filler = [torch.full((1 << 20,), 7, dtype=torch.uint8, device=gpu) for _ in range(8)]   # reuse of freed memory
    for _ in range(3):
        captured.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), "a replay after the workspace grew differs from the eager result"
        run_step(gpu, K2, V2, q2, q_pre2, k_new2, zT2.clone(), idx2, 8192, 1 / 16, False, workspace=ws)
        torch.cuda.synchronize()
    del filler
    assert int(ws.bytes(gpu, 0, "state").abs().sum()) == 0


def test_workspace_refuses_to_grow_under_capture(gpu):
    from attention_lab import _native as nat
    ws = nat.Workspace()
    ws.bytes(gpu, 1024, "t")
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with pytest.raises(RuntimeError, match="capture"):
            with torch.cuda.graph(g, stream=stream):
                ws.bytes(gpu, 1 << 24, "t")
    torch.cuda.synchronize()


def test_rejected_call_leaves_the_select_state_clean(gpu):
    """A call the select rejects (an unknown row order) must fail before the score kernel adds its histogram into the
    shared select state: the next valid call's rows are still bit-exact against the oracle."""
    from attention_lab import _native as nat
    from attention_lab import decode as dec
    B, G, h, C, L = 1, 8, 2, 2048 + 64, 2048
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=B, h=h, C=C, seed=31)
    req = prepare_request(B, G, C, valid_length=L, query_position=L - 1, rho=1 / 32, device=gpu)
    lo, hi, k, S = req.layout.candidate_lo, req.layout.candidate_hi, req.k, req.selected_count
    run_step(gpu, K, V, q, q_pre, k_pre_new, zT.clone(), idx, L, 1 / 32, False)   # sizes the module workspace
    ws = dec._STEP_WS.bytes(gpu, 0, "step")
    state = dec._STEP_WS.bytes(gpu, 0, "state")
    out = torch.empty(B, G, h, 128, dtype=torch.bfloat16, device=gpu)
    qm = q.reshape(B, G, h, 128).contiguous()
    qc = q_pre.reshape(B, G, h * 128).contiguous()
    kn = k_pre_new.reshape(B, G, 128).contiguous()
    with pytest.raises(ValueError, match="order"):
        nat.call("attnlab_sparse_decode_step", qm.data_ptr(), qc.data_ptr(), K.data_ptr(), V.data_ptr(),
                 zT.data_ptr(), idx.wq_t_scaled.data_ptr(), idx.wk.data_ptr(), kn.data_ptr(), B, G, h, 32, C, lo, hi,
                 L, k, L - 1, 0.088, 7, 1, state.data_ptr(), ws.data_ptr(), ws.numel(), None, None, out.data_ptr(),
                 nat.stream_of(gpu))
    torch.cuda.synchronize()
    assert int(state[:B * G * nat.SELECT_STATE_WORDS * 4].abs().sum()) == 0, "the rejected call touched the state"
    # a K the attend refuses (not 16-byte aligned), in position order with no row list (the one-launch select and
    # attend): refused before the score launch as well
    Kmis = torch.empty(K.numel() + 8, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="aligned"):
        nat.call("attnlab_sparse_decode_step", qm.data_ptr(), qc.data_ptr(), Kmis.data_ptr() + 2, V.data_ptr(),
                 zT.data_ptr(), idx.wq_t_scaled.data_ptr(), idx.wk.data_ptr(), kn.data_ptr(), B, G, h, 32, C, lo, hi,
                 L, k, L - 1, 0.088, nat.ORDER_POSITION, 1, state.data_ptr(), ws.data_ptr(), ws.numel(), None, None,
                 out.data_ptr(), nat.stream_of(gpu))
    torch.cuda.synchronize()
    assert int(state[:B * G * nat.SELECT_STATE_WORDS * 4].abs().sum()) == 0, "the rejected call touched the state"
    for canonical in (False, True):
        z = zT.clone()
        _, out2, pos = run_step(gpu, K, V, q, q_pre, k_pre_new, z, idx, L, 1 / 32, canonical)
        s = kernel_scores(z, q_pre, idx, lo, hi)
        want = exact.select_rows(s, lo, hi, L, k, order="position" if canonical else "score")
        assert np.array_equal(pos, want), f"canonical={canonical}: rows differ after a rejected call"


def test_a_fixed_set_other_than_the_rule_is_refused(gpu):
    """The step writes F from (lo, hi, legal) where the reference concatenates the fixed_rows it is given: any other
    set raises ValueError (select_rows_kernel and sparse_decode_step_kernel), an equal untagged copy is accepted."""
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=1, C=600, seed=12)
    L = 512
    req = prepare_request(1, 8, 600, valid_length=L, query_position=L - 1, rho=1 / 8, device=gpu)
    lo, hi, k, S = req.layout.candidate_lo, req.layout.candidate_hi, req.k, req.selected_count
    other = req.fixed_rows.clone()
    other[0, 0, 0] = other[0, 0, 0] + 7                               # a candidate row in place of position 0
    with pytest.raises(ValueError, match="selection rule"):
        sparse_decode_step_kernel(q, q_pre, K, V, zT, idx.wq_t_scaled, idx.wk, other, req.off_lo, lo, hi, k, S)
    with pytest.raises(ValueError, match="selection rule"):
        select_rows_kernel(idx.query(q_pre), zT, other, req.off_lo, lo, hi, k)
    a = sparse_decode_step_kernel(q, q_pre, K, V, zT, idx.wq_t_scaled, idx.wk, req.fixed_rows, req.off_lo, lo, hi, k, S)
    b = sparse_decode_step_kernel(q, q_pre, K, V, zT, idx.wq_t_scaled, idx.wk, req.fixed_rows.clone(),
                                  req.off_lo.clone(), lo, hi, k, S)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def _shape_scores(zT, lo, hi, case):
    """Candidate columns [lo, hi) of the index table rearranged so the score distribution stresses the list select:
    one tile far above the rest (its list cannot hold its share of the selection and the tile is read in full), every
    score equal (one first-digit bin holds the row: ties in index order, or the streaming select past 8192 keys), and
    seven distinct values (ties at the threshold across every list)."""
    M = hi - lo
    if case == "skewed_tile":
        zT[..., lo + M // 5: lo + M // 5 + 700] *= 4            # exact in bf16
        zT[..., hi - 300: hi] *= 2
    elif case == "all_equal":
        zT[..., lo:hi] = zT[..., lo:lo + 1].expand(*zT.shape[:-1], M)
    elif case == "seven_values":
        src = lo + (torch.arange(M, device=zT.device) * 5) % 7
        zT[..., lo:hi] = zT[..., src]
    else:
        raise ValueError(case)


@pytest.mark.parametrize("case", ["skewed_tile", "all_equal", "seven_values"])
@pytest.mark.parametrize("B,h,C,L,rho", [
    (2, 2, 8192 + 64, 8192, 1 / 8),       # one 512-column sub-tile per score workgroup, M < 8192
    (1, 2, 16384 + 64, 16384, 1 / 16),    # M > 8192: an all-equal row overflows the LDS candidates
    (16, 4, 16384, 16384, 1 / 32),        # two sub-tiles per score workgroup
])
def test_list_select_on_hard_distributions(gpu, case, B, h, C, L, rho):
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=B, h=h, C=C, seed=L + B)
    req0 = prepare_request(B, 8, C, valid_length=L, query_position=L - 1, rho=rho, device=gpu)
    lo, hi = req0.layout.candidate_lo, req0.layout.candidate_hi
    _shape_scores(zT, lo, hi, case)
    for canonical in (True, False):
        z = zT.clone()
        req, out, pos = run_step(gpu, K, V, q, q_pre, k_pre_new, z, idx, L, rho, canonical)
        k = req.k
        s = kernel_scores(z, q_pre, idx, lo, hi)
        want = exact.select_rows(s, lo, hi, L, k, order="position" if canonical else "score")
        assert np.array_equal(pos, want), f"{case} canonical={canonical}: row list differs from the oracle"
        if canonical:
            ref = exact.subset_attention(f64(q)[:, :, :, 0], f64(K), f64(V), want)
            check_out(out, ref, case)


@pytest.mark.parametrize("canonical", [True, False])
def test_list_select_state_is_left_clean(gpu, canonical):
    """After steps through the list select (including a row resolved by passes over its scores), a step with other
    shapes on the same select state is still bit-exact. Position order runs the fused select-and-attend (its
    workgroups share the state, the last reader clears it; h = 4 at B = 2 splits each row over head groups), score
    order the select kernel."""
    from attention_lab import decode as dec
    order = "position" if canonical else "score"
    for B, h, C, L, rho, case in ((1, 2, 16384 + 64, 16384, 1 / 16, "all_equal"), (2, 4, 8192 + 64, 8192, 1 / 8, None),
                                  (1, 2, 2048 + 64, 2048, 1 / 32, None)):
        K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=B, h=h, C=C, seed=C)
        req0 = prepare_request(B, 8, C, valid_length=L, query_position=L - 1, rho=rho, device=gpu)
        lo, hi = req0.layout.candidate_lo, req0.layout.candidate_hi
        if case:
            _shape_scores(zT, lo, hi, case)
        req, out, pos = run_step(gpu, K, V, q, q_pre, k_pre_new, zT, idx, L, rho, canonical)
        s = kernel_scores(zT, q_pre, idx, lo, hi)
        want = exact.select_rows(s, lo, hi, L, req.k, order=order)
        assert np.array_equal(pos, want)
        check_out(out, exact.subset_attention(f64(q)[:, :, :, 0], f64(K), f64(V), want), f"{order} {B}x{L}")
        state = dec._STEP_WS.bytes(gpu, 0, "state")
        assert int(state.abs().sum()) == 0, "the select left its state dirty"


@pytest.mark.parametrize("B,h,C,L,rho", [(1, 2, 2048 + 64, 2048, 1 / 32), (2, 4, 8192 + 64, 8192, 1 / 8),
                                         (16, 4, 32768, 32768, 1 / 32)])
def test_list_select_stages_through_the_abi(gpu, B, h, C, L, rho):
    """attnlab_score_grouped_lists + attnlab_select_lists, the two stages the step runs: scores equal the step's own
    score stage, rows are bit-exact against the oracle in both orders and equal the step's, and the state is left zero."""
    from attention_lab import _native as nat
    G = 8
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=B, h=h, C=C, seed=L + 7)
    req = prepare_request(B, G, C, valid_length=L, query_position=L - 1, rho=rho, device=gpu)
    lo, hi, k, S = req.layout.candidate_lo, req.layout.candidate_hi, req.k, req.selected_count
    M = hi - lo
    nbytes = nat.lib().attnlab_list_bytes(B, G, lo, hi, k, nat.ORDER_SCORE)
    assert nbytes > 0
    lists = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
    state = torch.zeros(B * G * nat.SELECT_STATE_WORDS, dtype=torch.int32, device=gpu)
    qc = q_pre.reshape(B, G, h * 128).contiguous()
    kn = k_pre_new.reshape(B, G, 128).contiguous()
    stream = nat.stream_of(gpu)
    for canonical in (True, False):
        order = nat.ORDER_POSITION if canonical else nat.ORDER_SCORE
        z = zT.clone()
        scores = torch.empty(B * G, M, dtype=torch.float32, device=gpu)
        rows = torch.empty(B * G, S, dtype=torch.int32, device=gpu)
        nat.call("attnlab_score_grouped_lists", z.data_ptr(), kn.data_ptr(), idx.wk.data_ptr(), qc.data_ptr(),
                 idx.wq_t_scaled.data_ptr(), None, scores.data_ptr(), M, B, G, 32, C, 128, h * 128, lo, hi, L - 1, k,
                 order, state.data_ptr(), lists.data_ptr(), nbytes, stream)
        nat.call("attnlab_select_lists", scores.data_ptr(), M, B, G, lo, hi, L, k, C, order, rows.data_ptr(), S, None,
                 state.data_ptr(), lists.data_ptr(), nbytes, None, 0, None, stream)
        torch.cuda.synchronize()
        assert int(state.abs().sum()) == 0, "the list select left its state dirty"
        s = scores.view(B, G, M).cpu().numpy()
        assert np.array_equal(s, kernel_scores(z, q_pre, idx, lo, hi)), "score stage differs from the step's"
        want = exact.select_rows(s, lo, hi, L, k, order="position" if canonical else "score")
        assert np.array_equal(rows.view(B, G, S).cpu().numpy(), want)
        _, _, pos = run_step(gpu, K, V, q, q_pre, k_pre_new, zT.clone(), idx, L, rho, canonical)
        assert np.array_equal(pos, want)


def test_step_without_select_state(gpu):
    """attnlab_sparse_decode_step with a null select state (the select then builds its own histograms) gives the rows
    and output of a step with one."""
    from attention_lab import _native as nat
    B, G, h, C, L = 2, 8, 2, 4096 + 64, 4096
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=B, h=h, C=C, seed=5)
    req = prepare_request(B, G, C, valid_length=L, query_position=L - 1, rho=1 / 16, device=gpu)
    lo, hi, k, S = req.layout.candidate_lo, req.layout.candidate_hi, req.k, req.selected_count
    ws_bytes = nat.lib().attnlab_sparse_decode_workspace(B, G, h, lo, hi, L, k, 1)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=gpu)
    state = torch.zeros(B * G * nat.SELECT_STATE_WORDS, dtype=torch.int32, device=gpu)
    qm = q.reshape(B, G, h, 128).contiguous()
    qc = q_pre.reshape(B, G, h * 128).contiguous()
    kn = k_pre_new.reshape(B, G, 128).contiguous()
    res = []
    for st in (state, None):
        z = zT.clone()
        out = torch.empty(B, G, h, 128, dtype=torch.bfloat16, device=gpu)
        rows = torch.empty(B * G, S, dtype=torch.int32, device=gpu)
        nat.call("attnlab_sparse_decode_step", qm.data_ptr(), qc.data_ptr(), K.data_ptr(), V.data_ptr(), z.data_ptr(),
                 idx.wq_t_scaled.data_ptr(), idx.wk.data_ptr(), kn.data_ptr(), B, G, h, 32, C, lo, hi, L, k, L - 1,
                 1 / np.sqrt(128), nat.ORDER_POSITION, 1, None if st is None else st.data_ptr(), ws.data_ptr(),
                 ws_bytes, rows.data_ptr(), None, out.data_ptr(), nat.stream_of(gpu))
        torch.cuda.synchronize()
        res.append((rows.cpu(), out.cpu()))
    assert int(state.abs().sum()) == 0
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])


def test_list_stages_refuse_score_order_past_the_lds_sort(gpu):
    """The list stages in score order past the LDS sort (k = 9830): attnlab_list_bytes gives 0 and the score stage
    refuses before it touches the select state; in position order the same k runs, bit-exact against the oracle, and
    leaves the state zero."""
    from attention_lab import _native as nat
    B, G, h, C, L = 1, 8, 2, 32768 + 64, 32768
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=B, h=h, C=C, seed=77)
    req = prepare_request(B, G, C, valid_length=L, query_position=L - 1, rho=0.3, device=gpu)
    lo, hi, k, S = req.layout.candidate_lo, req.layout.candidate_hi, req.k, req.selected_count
    assert k > nat.LDS_SORT_K
    M = hi - lo
    assert nat.lib().attnlab_list_bytes(B, G, lo, hi, k, nat.ORDER_SCORE) == 0
    nbytes = nat.lib().attnlab_list_bytes(B, G, lo, hi, k, nat.ORDER_POSITION)
    assert nbytes > 0, "the list select applies to this k in position order"
    lists = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
    state = torch.zeros(B * G * nat.SELECT_STATE_WORDS, dtype=torch.int32, device=gpu)
    qc = q_pre.reshape(B, G, h * 128).contiguous()
    stream = nat.stream_of(gpu)
    scores = torch.empty(B * G, M, dtype=torch.float32, device=gpu)
    rows = torch.empty(B * G, S, dtype=torch.int32, device=gpu)

    def score_stage(order):
        nat.call("attnlab_score_grouped_lists", zT.data_ptr(), None, idx.wk.data_ptr(), qc.data_ptr(),
                 idx.wq_t_scaled.data_ptr(), None, scores.data_ptr(), M, B, G, 32, C, 128, h * 128, lo, hi, L - 1, k,
                 order, state.data_ptr(), lists.data_ptr(), nbytes, stream)

    with pytest.raises(ValueError, match="score order"):
        score_stage(nat.ORDER_SCORE)
    torch.cuda.synchronize()
    assert int(state.abs().sum()) == 0, "the refused score stage touched the state"
    score_stage(nat.ORDER_POSITION)
    nat.call("attnlab_select_lists", scores.data_ptr(), M, B, G, lo, hi, L, k, C, nat.ORDER_POSITION, rows.data_ptr(),
             S, None, state.data_ptr(), lists.data_ptr(), nbytes, None, 0, None, stream)
    torch.cuda.synchronize()
    assert int(state.abs().sum()) == 0
    s = scores.view(B, G, M).cpu().numpy()
    assert np.array_equal(rows.view(B, G, S).cpu().numpy(), exact.select_rows(s, lo, hi, L, k, order="position"))


@pytest.mark.parametrize("case", [None, "skewed_tile", "all_equal"])
@pytest.mark.parametrize("B,h,C,L,rho", [(1, 2, 32768 + 64, 32768, 1 / 32), (16, 4, 16384, 16384, 1 / 32)])
def test_list_stages_without_stored_scores(gpu, case, B, h, C, L, rho):
    """The score stage writing key lists only (out NULL) and the list select recomputing what it needs from the table
    and u (an incomplete list's tile, a row resolved by radix passes): rows bit-exact against the oracle on the scores
    of the score kernel, equal to the same stages with stored scores, the state left zero."""
    from attention_lab import _native as nat
    G = 8
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=B, h=h, C=C, seed=L + B + 3)
    req = prepare_request(B, G, C, valid_length=L, query_position=L - 1, rho=rho, device=gpu)
    lo, hi, k, S = req.layout.candidate_lo, req.layout.candidate_hi, req.k, req.selected_count
    if case:
        _shape_scores(zT, lo, hi, case)
    M = hi - lo
    nbytes = nat.lib().attnlab_list_bytes(B, G, lo, hi, k, nat.ORDER_POSITION)
    lists = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
    state = torch.zeros(B * G * nat.SELECT_STATE_WORDS, dtype=torch.int32, device=gpu)
    u = torch.empty(B * G, 32, dtype=torch.float32, device=gpu)
    qc = q_pre.reshape(B, G, h * 128).contiguous()
    stream = nat.stream_of(gpu)
    got = []
    for stored in (False, True):
        scores = torch.empty(B * G, M, dtype=torch.float32, device=gpu) if stored else None
        rows = torch.empty(B * G, S, dtype=torch.int32, device=gpu)
        nat.call("attnlab_score_grouped_lists", zT.data_ptr(), None, idx.wk.data_ptr(), qc.data_ptr(),
                 idx.wq_t_scaled.data_ptr(), u.data_ptr(), nat.ptr(scores), M, B, G, 32, C, 128, h * 128, lo, hi, L - 1,
                 k, nat.ORDER_POSITION, state.data_ptr(), lists.data_ptr(), nbytes, stream)
        nat.call("attnlab_select_lists", nat.ptr(scores), M, B, G, lo, hi, L, k, C, nat.ORDER_POSITION,
                 rows.data_ptr(), S, None, state.data_ptr(), lists.data_ptr(), nbytes, zT.data_ptr(), nat.DT_BF16,
                 u.data_ptr(), stream)
        torch.cuda.synchronize()
        assert int(state.abs().sum()) == 0, f"stored={stored}: the list select left its state dirty"
        got.append(rows.view(B, G, S).cpu().numpy())
    s = kernel_scores(zT, q_pre, idx, lo, hi)
    want = exact.select_rows(s, lo, hi, L, k, order="position")
    assert np.array_equal(got[0], want), "recomputed scores: row list differs from the oracle"
    assert np.array_equal(got[1], want)


@pytest.mark.parametrize("G,h,P", [(3, 2, 3), (3, 2, 8), (8, 2, 5), (8, 4, 16), (1, 2, 8)])
def test_in_kernel_partition_merge_equals_the_combine_kernel(gpu, G, h, P):
    """The step merges its split-K partials inside the attend kernel (the last partition workgroup to arrive, counted
    in the select state). Grids of 3 x 2 x 3 or 3 x 2 x 8 workgroups put a (b, g)'s partitions on several XCDs. Two
    calls with different queries: each output equals, bit for bit, attnlab_attend with the combine kernel over the
    same rows and partitions, and meets the bf16 bar against the float64 oracle; the state is left zero."""
    from attention_lab import _native as nat
    B, C, L = 1, 8192 + 64, 8192
    ws = nat.Workspace()
    for call in range(2):
        K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=B, G=G, h=h, C=C, seed=100 + 10 * G + call)
        req = prepare_request(B, G, C, valid_length=L, query_position=L - 1, rho=1 / 8, device=gpu)
        out, flat = sparse_decode_step_kernel(q, q_pre, K, V, zT, idx.wq_t_scaled, idx.wk, req.fixed_rows, req.off_lo,
                                              req.layout.candidate_lo, req.layout.candidate_hi, req.k,
                                              req.selected_count, k_pre_new=k_pre_new, write_col=req.write_col,
                                              return_rows=True, canonical_order=True, partitions=P, workspace=ws)
        torch.cuda.synchronize()
        S = req.selected_count
        pos = (flat.view(B, G, S) - req.offsets).to(torch.int32).contiguous()
        ref = hip_attend.attend(q.reshape(B, G, h, 128).contiguous(), K, V, pos, partitions=P)
        torch.cuda.synchronize()
        assert torch.equal(out.view(B, G, h, 128), ref), f"call {call}: in-kernel merge differs from the combine kernel"
        want = exact.subset_attention(f64(q)[:, :, :, 0], f64(K), f64(V), pos.cpu().numpy())
        check_out(out, want, f"G={G} P={P} call {call}")
        assert int(ws.bytes(gpu, 0, "state").abs().sum()) == 0, "arrival counters left non-zero"


@pytest.mark.parametrize("B,G,h,C,L,rho,case,P", [
    (1, 8, 2, 2048 + 64, 2048, 1 / 32, None, None),          # config 1
    (1, 8, 2, 32768 + 64, 32768, 1 / 32, None, None),        # B=1 at 32K: partitions split each row
    (16, 8, 4, 16384, 16384, 1 / 32, None, None),            # two sub-tiles per score workgroup
    (2, 8, 4, 8192 + 64, 8192, 1 / 8, "skewed_tile", None),  # an incomplete list: its tile recomputed
    (1, 8, 2, 16384 + 64, 16384, 1 / 16, "all_equal", None), # bin b1 past the LDS candidates: radix passes
    (2, 8, 2, 8192 + 64, 8192, 1 / 8, "seven_values", None), # ties at the threshold
    (1, 3, 2, 8192 + 64, 8192, 1 / 8, None, 1),
    (1, 3, 2, 8192 + 64, 8192, 1 / 8, None, 3),              # partitions of one row on several XCDs
    (1, 3, 4, 8192 + 64, 8192, 1 / 8, None, 16),
    (1, 2, 1, 300, 256, 1 / 8, None, None),                  # sinks, picks and recent rows in one partition
    (1, 8, 2, 2048 + 64, 2048, 1 / 32, None, 64),            # S = 132 over 64 partitions: 20 of them empty
    (1, 8, 6, 2048 + 64, 2048, 1 / 32, None, None),          # three heads per workgroup: the separate launches
    (2, 4, 3, 4096 + 64, 4096, 1 / 16, None, 4),             # likewise, odd h
])
def test_fused_select_attend_equals_the_separate_stages(gpu, B, G, h, C, L, rho, case, P):
    """A step whose row list does not leave the call selects and attends in one launch (every workgroup of a row
    repeats the row's selection and keeps its partition of the row list in LDS). Its output equals, bit for bit, the
    same step run as separate select and attend launches (asking for the rows) in position order, twice in a row on one
    workspace with other queries; the select state is zero after each call."""
    from attention_lab import _native as nat
    ws = nat.Workspace()
    K, V, q, q_pre, k_pre_new, zT, idx = setup(gpu, B=B, G=G, h=h, C=C, seed=L + B + G + h)
    req = prepare_request(B, G, C, valid_length=L, query_position=L - 1, rho=rho, device=gpu)
    lo, hi = req.layout.candidate_lo, req.layout.candidate_hi
    if case:
        _shape_scores(zT, lo, hi, case)
    for call in range(2):
        if call:
            q = torch.randn(q.shape, generator=torch.Generator().manual_seed(call)).to(torch.bfloat16).to(gpu)
        outs = []
        for rows in (False, True):
            z = zT.clone()
            got = sparse_decode_step_kernel(q, q_pre, K, V, z, idx.wq_t_scaled, idx.wk, req.fixed_rows, req.off_lo,
                                            lo, hi, req.k, req.selected_count, k_pre_new=k_pre_new,
                                            write_col=req.write_col, return_rows=rows, canonical_order=True,
                                            partitions=P, workspace=ws)
            torch.cuda.synchronize()
            assert int(ws.bytes(gpu, 0, "state").abs().sum()) == 0, f"rows={rows}: the select state left dirty"
            outs.append(got[0] if rows else got)
        assert torch.equal(outs[0], outs[1]), f"call {call}: the fused launch differs from the separate stages"
    s = kernel_scores(zT, q_pre, idx, lo, hi)
    want = exact.select_rows(s, lo, hi, L, req.k, order="position")
    check_out(outs[0], exact.subset_attention(f64(q)[:, :, :, 0], f64(K), f64(V), want), f"{case} P={P}")
