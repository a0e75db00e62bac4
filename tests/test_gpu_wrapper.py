"""The Qwen3 wrapper on the HIP path (reference tests/test_qwen_wrapper.py:117-500, on a bf16 tiny Qwen3 with head_dim
128 so every read runs on this build's kernels).

The unmodified model, the comparison target, runs on the CPU in bf16 with the same weights: its attention (torch
SDPA) is outside this build and bf16 batched products on the GPU are avoided in references. Tolerances are the
reference's bf16 contract tolerances (atol 5e-2, relative norm 2e-2), except that "same path, same inputs" checks are
exact. Invariants from the reference: every candidate selected equals the full read; poisoning every row a sparse
step did not select changes nothing while the full read sees it; unwritten, future and rolled-back slots are never
read; chunked prefill equals one shot; the phase is explicit and a prefill chunk never selects.
"""
from __future__ import annotations

import copy

import pytest
import torch

transformers = pytest.importorskip("transformers")
from transformers import DynamicCache  # noqa: E402

from attention_lab.qwen_wrap import (LabRunner, NativeRunner, hf_cache_kv, is_wrapped, make_state,  # noqa: E402
                                     tiny_qwen3, unwrap_model, wrap_model)
from attention_lab.selection import fixed_budget  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = {"atol": 5e-2, "rel_norm": 2e-2}
EXACT = {"atol": 0.0, "rel_norm": 0.0}
VOCAB = 256


def tiny_pair(gpu, seed=0):
    """The same random-init Qwen3 twice: bf16 on the GPU (to be wrapped) and bf16 on the CPU (the reference)."""
    cpu = tiny_qwen3(seed=seed, layers=2, hidden=256, heads=4, groups=2, head_dim=128, intermediate=256, vocab=VOCAB,
                     dtype=torch.bfloat16)
    return copy.deepcopy(cpu).to(gpu), cpu


def token_ids(n, seed=0):
    return torch.randint(0, VOCAB, (1, n), generator=torch.Generator().manual_seed(1000 + seed))


def assert_close(a, b, tol, what):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    assert a.shape == b.shape, f"{what}: shape {tuple(a.shape)} vs {tuple(b.shape)}"
    assert torch.isfinite(a).all(), f"{what}: non-finite values"
    d = (a - b).abs()
    rel = float(d.norm() / b.norm().clamp_min(1e-30))
    assert float(d.max()) <= tol["atol"] and rel <= tol["rel_norm"], f"{what}: max {float(d.max()):.3e} rel {rel:.3e}"


def poison_unwritten(cache):
    L = cache.valid_length
    for l in range(cache.layers):
        cache.k[l][:, :, L:] = float("nan")
        cache.v[l][:, :, L:] = float("nan")
        if cache.z is not None:
            cache.z[l][..., L:] = float("nan")


@pytest.mark.parametrize("L", [32, 128, 300])
def test_full_path_matches_the_unmodified_model_and_its_cache(gpu, L):
    m, ref_model = tiny_pair(gpu)
    ids = token_ids(L)
    with torch.inference_mode():
        ref = ref_model(ids).logits
        dc = DynamicCache(config=ref_model.config)
        ref_model(ids, past_key_values=dc, use_cache=True)
        holder = wrap_model(m)
        st = make_state(m, L + 40, "full")
        run = LabRunner(m, holder, st)
        poison_unwritten(st.cache)
        one_shot = run.prefill(ids.to(gpu), L, keep_logits=True)
        assert_close(one_shot, ref, TOL, "wrapped one-shot prefill vs unmodified logits")
        for l in range(st.cache.layers):
            k, v = hf_cache_kv(dc, l)
            assert_close(st.cache.k[l][:, :, :L], k, TOL, f"layer {l} K: static cache vs transformers cache")
            assert_close(st.cache.v[l][:, :, :L], v, TOL, f"layer {l} V: static cache vs transformers cache")
        st2 = make_state(m, L + 40, "full")
        run2 = LabRunner(m, holder, st2)
        poison_unwritten(st2.cache)
        head = run2.prefill(ids[:, :L - 8].to(gpu), 37, keep_logits=True)
        tail = torch.cat([run2.step(ids[:, i:i + 1].to(gpu)) for i in range(L - 8, L)], dim=1)
        assert_close(torch.cat([head, tail], 1), ref, TOL, "wrapped incremental vs unmodified logits")
        assert st2.cache.valid_length == L
        assert st2.cache.writes == [-(-(L - 8) // 37) + 8] * st2.cache.layers, "one append per layer per forward"
        unwrap_model(m)
        assert not is_wrapped(m)


def test_every_candidate_selected_matches_full_and_unselected_rows_are_never_read(gpu):
    m, ref_model = tiny_pair(gpu, seed=1)
    L = 160
    ids = token_ids(L, seed=2)
    with torch.inference_mode():
        ref = ref_model(ids).logits
        ids = ids.to(gpu)
        holder = wrap_model(m)
        stA = make_state(m, L + 16, "full")
        runA = LabRunner(m, holder, stA)
        runA.prefill(ids[:, :L - 6], 50)
        stD = make_state(m, L + 16, "sparse")
        runD = LabRunner(m, holder, stD)
        runD.prefill(ids[:, :L - 6], 50)
        stD.begin_request(None, k0=stD.cache.capacity)              # every candidate on every step
        outA, outD = [], []
        for i in range(L - 6, L):
            outA.append(runA.step(ids[:, i:i + 1]))
            outD.append(runD.step(ids[:, i:i + 1]))
            assert stD.plan.selected_count == stD.plan.legal_length
        outA, outD = torch.cat(outA, 1), torch.cat(outD, 1)
        assert_close(outA, ref[:, L - 6:], TOL, "wrapped full decode vs unmodified")
        assert_close(outD, outA, TOL, "sparse read with every position selected vs full read")
        # a partial read: poison every row the step did not select, in both caches -> D unchanged, A broken
        runD.rollback(L - 6)
        runA.rollback(L - 6)
        stD.begin_request(1 / 8)
        assert stD.k0 == fixed_budget(L - 5, 1 / 8)
        stD.record_selection = True
        clean = runD.step(ids[:, L - 6:L - 5])
        plan = stD.plan
        assert plan.selected_count < plan.legal_length
        C, G = stD.cache.capacity, stD.cache.groups
        for l in range(stD.cache.layers):
            rows = stD.last_rows[l].view(1, G, plan.selected_count) - stD.cache.offsets
            assert rows.min() >= 0 and rows.max() < plan.legal_length
            for g in range(G):
                keep = torch.zeros(C, dtype=torch.bool, device=gpu)
                keep[rows[0, g]] = True
                for cache in (stD.cache, stA.cache):
                    cache.k[l][0, g, ~keep] = float("nan")
                    cache.v[l][0, g, ~keep] = float("nan")
        runD.rollback(L - 6)
        poisoned = runD.step(ids[:, L - 6:L - 5])
        assert torch.isfinite(poisoned).all(), "the sparse read touched a row it did not select"
        assert_close(poisoned, clean, EXACT, "sparse step with its unselected rows poisoned")
        assert not torch.isfinite(runA.step(ids[:, L - 6:L - 5])).all(), "the full read must see the poison"
        unwrap_model(m)


@pytest.mark.parametrize("mode,selector", [("full", "index"), ("sparse", "index"), ("sparse", "recent"),
                                           ("sparse", "uniform")])
def test_unwritten_and_future_slots_never_change_a_step(gpu, mode, selector):
    m, _ = tiny_pair(gpu, seed=3)
    L = 120
    ids = token_ids(L, seed=3).to(gpu)
    with torch.inference_mode():
        holder = wrap_model(m)
        st = make_state(m, L + 64, mode, selector=selector)
        run = LabRunner(m, holder, st)
        run.prefill(ids[:, :L - 5], 40)
        if mode == "sparse":
            st.begin_request(1 / 8)
        clean = torch.cat([run.step(ids[:, i:i + 1]) for i in range(L - 5, L)], 1)
        run.rollback(L - 5)
        for l in range(st.cache.layers):       # garbage and a huge finite value in the future slots
            st.cache.k[l][:, :, L - 5:L - 2] = float("nan")
            st.cache.k[l][:, :, L - 2:] = 1e6
            st.cache.v[l][:, :, L - 5:] = float("nan")
            if st.cache.z is not None:
                st.cache.z[l][..., L - 5:] = float("nan")
        again = torch.cat([run.step(ids[:, i:i + 1]) for i in range(L - 5, L)], 1)
        assert_close(again, clean, EXACT, f"{mode}/{selector}: poisoned future slots")
        unwrap_model(m)


@pytest.mark.parametrize("mode", ["full", "sparse"])
def test_rollback_replays_and_the_old_suffix_is_unreadable(gpu, mode):
    m, _ = tiny_pair(gpu, seed=4)
    ids, alt = token_ids(140, seed=4).to(gpu), token_ids(140, seed=5).to(gpu)
    with torch.inference_mode():
        holder = wrap_model(m)
        st = make_state(m, 160, mode)
        run = LabRunner(m, holder, st)
        run.prefill(ids[:, :100], 37)
        if mode == "sparse":
            st.begin_request(1 / 8)
        first = torch.cat([run.step(ids[:, i:i + 1]) for i in range(100, 105)], 1)
        assert st.cache.valid_length == 105
        run.rollback(100)
        poison_unwritten(st.cache)
        second = torch.cat([run.step(ids[:, i:i + 1]) for i in range(100, 105)], 1)
        assert_close(second, first, EXACT, f"{mode}: same tokens after a rollback")
        run.rollback(100)
        branch = torch.cat([run.step(alt[:, i:i + 1]) for i in range(100, 105)], 1)
        fresh = make_state(m, 160, mode)
        runf = LabRunner(m, holder, fresh)
        runf.prefill(ids[:, :100], 100)
        if mode == "sparse":
            fresh.begin_request(1 / 8)
        fresh_out = torch.cat([runf.step(alt[:, i:i + 1]) for i in range(100, 105)], 1)
        assert_close(branch, fresh_out, TOL, f"{mode}: overwritten suffix vs a fresh cache")
        with pytest.raises(ValueError):
            run.rollback(200)
        unwrap_model(m)


def test_chunked_prefill_matches_one_shot_for_kv_and_index_table(gpu):
    m, _ = tiny_pair(gpu, seed=6)
    L = 100
    ids = token_ids(L, seed=6).to(gpu)
    with torch.inference_mode():
        holder = wrap_model(m)
        one = make_state(m, L + 8, "sparse")
        LabRunner(m, holder, one).prefill(ids, L)
        chunked = make_state(m, L + 8, "sparse")
        runc = LabRunner(m, holder, chunked)
        for a, b in zip([0, 5, 50], [5, 50, 100]):
            runc.forward(ids[:, a:b], phase="prefill", logits_to_keep=1)
        assert chunked.cache.valid_length == L
        for l in range(one.cache.layers):
            assert_close(chunked.cache.k[l][:, :, :L], one.cache.k[l][:, :, :L], TOL, f"layer {l} K")
            assert_close(chunked.cache.v[l][:, :, :L], one.cache.v[l][:, :, :L], TOL, f"layer {l} V")
            assert_close(chunked.cache.z[l][..., :L], one.cache.z[l][..., :L], TOL, f"layer {l} z")
        unwrap_model(m)


def test_k_rule_fixed_per_request_and_short_history_reads_everything(gpu):
    m, _ = tiny_pair(gpu, seed=7)
    ids = token_ids(200, seed=7).to(gpu)
    with torch.inference_mode():
        holder = wrap_model(m)
        # short history (legal < 68): the sparse read is the full read
        stA, stD = make_state(m, 80, "full"), make_state(m, 80, "sparse")
        runA, runD = LabRunner(m, holder, stA), LabRunner(m, holder, stD)
        runA.prefill(ids[:, :40], 40)
        runD.prefill(ids[:, :40], 40)
        stD.begin_request(1 / 8)
        a = torch.cat([runA.step(ids[:, i:i + 1]) for i in range(40, 50)], 1)
        d = torch.cat([runD.step(ids[:, i:i + 1]) for i in range(40, 50)], 1)
        assert stD.plan.k == 0 and stD.plan.selected_count == stD.plan.legal_length
        assert_close(d, a, TOL, "short history: sparse vs full")
        # k0 is fixed by the request's first legal length and clamped per step
        st = make_state(m, 260, "sparse")
        run = LabRunner(m, holder, st)
        run.prefill(ids[:, :150], 64)
        k0 = st.begin_request(1 / 8)
        assert k0 == fixed_budget(151, 1 / 8)
        for i in range(150, 160):
            run.step(ids[:, i:i + 1])
            assert st.plan.k0 == k0 and st.plan.k == min(k0, st.plan.legal_length - 68)
        unwrap_model(m)


def test_phase_is_explicit_and_prefill_never_selects(gpu):
    m, _ = tiny_pair(gpu, seed=8)
    ids = token_ids(120, seed=8).to(gpu)
    with torch.inference_mode():
        holder = wrap_model(m)
        st = make_state(m, 160, "sparse")
        run = LabRunner(m, holder, st)
        with pytest.raises(ValueError):
            run.forward(ids[:, :4], phase="chunk")
        with pytest.raises(ValueError):
            run.step(ids[:, :2])
        run.prefill(ids[:, :100], 64)
        with pytest.raises(RuntimeError):        # no request begun (raised before any layer runs)
            run.step(ids[:, 100:101])
        assert st.cache.valid_length == 100
        st.begin_request(1 / 8)
        st.record_selection = True
        run.forward(ids[:, 100:101], phase="prefill")   # a one-token prefill chunk reads everything, selects nothing
        assert st.plan is None and all(r is None for r in st.last_rows)
        run.step(ids[:, 101:102])
        assert all(r is not None for r in st.last_rows)
        unwrap_model(m)


@pytest.mark.parametrize("selector", ["recent", "uniform"])
def test_recent_and_uniform_selectors(gpu, selector):
    m, _ = tiny_pair(gpu, seed=9)
    L = 200
    ids = token_ids(L, seed=9).to(gpu)
    with torch.inference_mode():
        holder = wrap_model(m)
        stA = make_state(m, L + 8, "full")
        runA = LabRunner(m, holder, stA)
        runA.prefill(ids[:, :150], 64)
        st = make_state(m, L + 8, "sparse", selector=selector, uniform_seed=5)
        assert st.cache.z is None and st.indexers is None
        run = LabRunner(m, holder, st)
        run.prefill(ids[:, :150], 64)
        st.begin_request(1 / 8)
        st.record_selection = True
        first = run.step(ids[:, 150:151])
        plan = st.plan
        rows = st.last_rows[0].view(1, st.cache.groups, plan.selected_count) - st.cache.offsets
        fixed = list(range(4)) + list(range(plan.hi, plan.legal_length))
        for g in range(st.cache.groups):
            got = sorted(rows[0, g].tolist())
            assert set(fixed) <= set(got) and len(set(got)) == plan.selected_count
            cands = [p for p in got if plan.lo <= p < plan.hi]
            if selector == "recent":
                assert cands == list(range(plan.hi - plan.k, plan.hi))
        # the same (request, step) after a rollback draws the same rows and gives the same logits
        rows0 = st.last_rows[0].clone()
        run.rollback(150)
        again = run.step(ids[:, 150:151])
        assert torch.equal(st.last_rows[0], rows0)
        assert_close(again, first, EXACT, f"{selector}: replay after rollback")
        # every candidate selected: the full read
        run.rollback(150)
        st.begin_request(None, k0=st.cache.capacity)
        d = run.step(ids[:, 150:151])
        a = runA.step(ids[:, 150:151])
        assert_close(d, a, TOL, f"{selector} with every candidate vs full")
        unwrap_model(m)


def test_native_runner_matches_the_unmodified_model_and_rolls_back():
    """NativeRunner (transformers' own cache) is the wrapper's comparison target; checked on the CPU."""
    _, m = tiny_pair("cpu", seed=10)
    ids = token_ids(60, seed=10)
    with torch.inference_mode():
        ref = m(ids).logits
        run = NativeRunner(m, DynamicCache(config=m.config), 80)
        head = run.prefill(ids[:, :50], 16, keep_logits=True)
        tail = torch.cat([run.step(ids[:, i:i + 1]) for i in range(50, 60)], 1)
        assert_close(torch.cat([head, tail], 1), ref, TOL, "native incremental vs one shot")
        run.rollback(50)
        again = torch.cat([run.step(ids[:, i:i + 1]) for i in range(50, 60)], 1)
        assert_close(again, tail, TOL, "native replay after rollback")


@pytest.mark.parametrize("canonical", [False, True])
def test_every_candidate_at_32k_in_either_row_order_equals_the_full_read(gpu, canonical):
    """k0 = capacity at a 32K context selects ~32.7K candidates per step: score order (the wrapper's default, its
    radix pass) and position order must both read exactly the full legal range and match the full read (reference
    tests/test_qwen_wrapper.py:150-173)."""
    m, _ = tiny_pair(gpu, seed=11)
    L = 32768
    ids = token_ids(L + 3, seed=11).to(gpu)
    with torch.inference_mode():
        holder = wrap_model(m)
        stA = make_state(m, L + 8, "full")
        runA = LabRunner(m, holder, stA)
        runA.prefill(ids[:, :L], 8192)
        stD = make_state(m, L + 8, "sparse", canonical_order=canonical)
        runD = LabRunner(m, holder, stD)
        runD.prefill(ids[:, :L], 8192)
        stD.begin_request(None, k0=stD.cache.capacity)
        stD.record_selection = True
        for i in range(L, L + 3):
            a = runA.step(ids[:, i:i + 1])
            d = runD.step(ids[:, i:i + 1])
            plan = stD.plan
            assert plan.k == plan.candidate_count > 8192 and plan.selected_count == plan.legal_length
            rows = stD.last_rows[0].view(1, stD.cache.groups, plan.selected_count) - stD.cache.offsets
            assert torch.equal(rows.sort(dim=-1).values[0, 0].cpu(), torch.arange(plan.legal_length))
            if canonical:
                assert torch.equal(rows[0, 0].cpu(), torch.arange(plan.legal_length))
            assert_close(d, a, TOL, f"step {i}: every candidate ({'position' if canonical else 'score'} order) vs full")
        unwrap_model(m)


def test_a_sparse_step_runs_one_select_per_layer_and_no_dense_read(gpu, monkeypatch):
    """The reference spies on a model step: one torch.topk per layer and no torch.gather in a sparse step, no top-k in
    a full one (tests/test_qwen_wrapper.py:324-345), and its profiler check finds no full-length QK in the sparse read
    (bench/microbench.py:207-229). Here every read is a C-ABI call, so the spy counts the entry points a step reaches:
    a sparse step makes exactly one fused call per layer (its one select launch inside), and no dense decode, prefill,
    standalone select, torch.topk, torch.gather or full_attention; a full step makes one dense decode per layer and no
    sparse call. Both steps also rerun with the spy off and give the same logits."""
    from attention_lab import _native as nat
    from attention_lab import full as full_mod
    from attention_lab import qwen_wrap
    m, _ = tiny_pair(gpu, seed=6)
    ids = token_ids(140, seed=6).to(gpu)
    calls = []
    real_call = nat.call

    def spy(name, *args):
        calls.append(name)
        return real_call(name, *args)

    def refuse(*a, **k):
        raise AssertionError("the sparse step took a dense read")

    with torch.inference_mode():
        holder = wrap_model(m)
        st = make_state(m, 160, "sparse")
        run = LabRunner(m, holder, st)
        run.prefill(ids[:, :129], 129)
        st.begin_request(1 / 8)
        with monkeypatch.context() as mp:
            mp.setattr(nat, "call", spy)
            mp.setattr(qwen_wrap, "full_attention", refuse)
            mp.setattr(full_mod, "full_attention", refuse)
            mp.setattr(torch, "topk", lambda *a, **k: (_ for _ in ()).throw(AssertionError("torch.topk in a step")))
            mp.setattr(torch, "gather", lambda *a, **k: (_ for _ in ()).throw(AssertionError("torch.gather in a step")))
            spied = run.step(ids[:, 129:130])
        layers = st.cache.layers
        assert calls.count("attnlab_sparse_decode_step") == layers, calls
        assert set(calls) == {"attnlab_sparse_decode_step"}, f"a sparse step reached {sorted(set(calls))}"
        assert st.plan.selected_count < st.plan.legal_length, "the step must be a partial read"
        run.rollback(129)
        torch.testing.assert_close(run.step(ids[:, 129:130]), spied, rtol=0, atol=0)

        calls.clear()
        stA = make_state(m, 160, "full")
        runA = LabRunner(m, holder, stA)
        runA.prefill(ids[:, :129], 129)
        with monkeypatch.context() as mp:
            mp.setattr(nat, "call", spy)
            runA.step(ids[:, 129:130])
        assert calls.count("attnlab_dense_decode") == layers, calls
        assert "attnlab_sparse_decode_step" not in calls and not any("select" in c or "topk" in c for c in calls)
        unwrap_model(m)
