"""Host-side contracts of the Qwen3 wrapper (no kernel call): the static cache's append / advance / rollback / clone
ledger, the step plan, the state's validation and the geometry read from a model (reference
tests/test_qwen_wrapper.py:109-115 and qwen_wrap.py:52-256). Skipped without transformers."""
from __future__ import annotations

import pytest
import torch

transformers = pytest.importorskip("transformers")

from attention_lab.qwen_wrap import (LabCache, LabState, StateHolder, build_step_plan, geometry_of,  # noqa: E402
                                     is_wrapped, make_cache, tiny_qwen3, unwrap_model, wrap_model)
from attention_lab.selection import fixed_budget  # noqa: E402


def cache(**kw):
    args = dict(layers=2, batch=2, groups=2, capacity=300, head_dim=4, index_dim=3, device="cpu", dtype=torch.float32)
    args.update(kw)
    return LabCache(**args)


def test_geometry_comes_from_config_and_matches_parameters():
    m = tiny_qwen3()
    geo = geometry_of(m)
    assert (geo.layers, geo.hidden, geo.heads, geo.groups, geo.head_dim, geo.heads_per_group) == (2, 64, 4, 2, 16, 2)
    m.config.num_key_value_heads = 4   # no longer matches k_proj: must be detected
    with pytest.raises(ValueError):
        geometry_of(m)


def test_wrap_unwrap_keeps_the_original_modules():
    m = tiny_qwen3()
    inner = [layer.self_attn for layer in m.model.layers]
    holder = wrap_model(m)
    assert isinstance(holder, StateHolder) and is_wrapped(m)
    assert [layer.self_attn.inner for layer in m.model.layers] == inner
    with pytest.raises(RuntimeError):
        wrap_model(m)
    unwrap_model(m)
    assert not is_wrapped(m) and [layer.self_attn for layer in m.model.layers] == inner


def test_append_advance_and_rollback_ledger():
    c = cache()
    assert c.has_index and c.valid_length == 0
    k = torch.randn(2, 2, 5, 4)
    z = torch.randn(2, 2, 3, 5)
    for layer in range(2):
        c.append(layer, k, k + 1, z)
    c.advance(5)
    assert c.valid_length == 5 and c.writes == [1, 1] and c.last_write == [(0, 5), (0, 5)]
    assert torch.equal(c.k[1][:, :, :5], k) and torch.equal(c.v[0][:, :, :5], k + 1)
    assert torch.equal(c.z[0][..., :5], z)
    c.append(0, k[:, :, :2], k[:, :, :2])
    with pytest.raises(RuntimeError):          # another length in the same forward
        c.append(1, k, k)
    with pytest.raises(RuntimeError):          # not every layer appended
        c.advance(2)
    with pytest.raises(RuntimeError):          # rollback while a forward is in flight
        c.rollback(3)
    c.append(1, k[:, :, :2], k[:, :, :2])
    c.advance(2)
    assert c.valid_length == 7
    c.rollback(3)
    assert c.valid_length == 3
    with pytest.raises(ValueError):
        c.rollback(4)
    with pytest.raises(RuntimeError):          # capacity
        c.append(0, torch.zeros(2, 2, 298, 4), torch.zeros(2, 2, 298, 4))
    no_index = cache(index_dim=None)
    with pytest.raises(RuntimeError):
        no_index.append(0, k, k, z)


def test_clone_shares_no_storage_and_bytes_ledger():
    c = cache()
    c.append(0, torch.ones(2, 2, 1, 4), torch.ones(2, 2, 1, 4))
    c.append(1, torch.ones(2, 2, 1, 4), torch.ones(2, 2, 1, 4))
    c.advance(1)
    d = c.clone()
    d.k[0].zero_()
    assert float(c.k[0][0, 0, 0, 0]) == 1.0 and d.valid_length == 1 and d.writes == c.writes
    b = c.bytes()
    # capacity 300 is held as 304 slots per (b, g) (a multiple of 8)
    assert b["kv_bytes"] == 2 * 2 * 2 * 2 * 304 * 4 * 4 and b["index_bytes"] == 2 * 2 * 2 * 3 * 304 * 4
    assert b["total_bytes"] == b["kv_bytes"] + b["index_bytes"]


@pytest.mark.parametrize("legal", [300, 100, 68, 40])
def test_step_plan_follows_the_selection_rules(legal):
    c = cache()
    k0 = fixed_budget(100, 1 / 8)
    plan = build_step_plan(c, legal, k0)
    assert plan.write_col == legal - 1
    pos = plan.fixed_rows - c.offsets
    assert tuple(pos.shape[:2]) == (2, 2)
    if legal >= 68:
        assert (plan.lo, plan.hi) == (4, legal - 64)
        assert pos[0, 0].tolist() == list(range(4)) + list(range(legal - 64, legal))
        assert plan.k == min(k0, legal - 68) and plan.selected_count == 68 + plan.k
    else:   # short history: F covers every legal position, nothing is selected
        assert plan.k == 0 and plan.selected_count == legal == plan.fixed_count
        assert pos[1, 1].tolist() == list(range(legal))
    assert torch.equal(plan.off_lo - c.offsets, torch.full_like(plan.off_lo, plan.lo))


def test_state_validation():
    c = cache()
    with pytest.raises(ValueError):
        LabState(c, mode="dense")
    with pytest.raises(ValueError):
        LabState(c, mode="sparse", selector="topk")
    with pytest.raises(ValueError):           # D0 needs indexers
        LabState(c, mode="sparse")
    with pytest.raises(ValueError):
        LabState(c, [object()], mode="full")
    with pytest.raises(ValueError):
        LabState(c, mode="full", sparse_layers=[2])
    st = LabState(cache(index_dim=None), mode="sparse", selector="recent")
    c2 = st.cache
    c2.append(0, torch.zeros(2, 2, 99, 4), torch.zeros(2, 2, 99, 4))
    c2.append(1, torch.zeros(2, 2, 99, 4), torch.zeros(2, 2, 99, 4))
    c2.advance(99)
    assert st.begin_request(1 / 8) == fixed_budget(100, 1 / 8) and st.request_start_length == 100
    assert st.begin_request(None, k0=300) == 300 and st.request_counter == 2
    a, b = st.uniform_rng(3).random(4), st.uniform_rng(3).random(4)
    assert (a == b).all()


def test_make_cache_takes_the_model_geometry():
    m = tiny_qwen3(dtype=torch.float32)
    c = make_cache(m, 50, with_index=True, index_dim=8, batch=3)
    assert (c.layers, c.batch, c.groups, c.capacity, c.head_dim, c.index_dim) == (2, 3, 2, 50, 16, 8)
    # rows in memory: the capacity rounded up to 8 (16-byte index-table rows); the bytes count what is held
    assert c.slots == 56 and tuple(c.k[0].shape) == (3, 2, 56, 16)
    assert c.k[0].dtype == torch.float32 and tuple(c.z[1].shape) == (3, 2, 8, 56)
    assert c.bytes()["total_bytes"] == sum(t.numel() * t.element_size() for t in c.k + c.v + c.z)


def test_fixed_set_check_accepts_the_rule_and_refuses_anything_else():
    """The HIP step writes F from (lo, hi, legal): the rule's F (tagged by prepare_request, or equal by value) passes,
    any other fixed_rows / off_lo raises ValueError instead of being silently replaced."""
    import torch
    from attention_lab.decode import check_standard_f, prepare_request
    req = prepare_request(2, 3, 300, valid_length=256, query_position=255, rho=1 / 8, device="cpu")
    lo, hi, legal = req.layout.candidate_lo, req.layout.candidate_hi, req.layout.legal_length
    check_standard_f(req.fixed_rows, req.off_lo, lo, hi, legal, 300)                  # tagged: no device read
    check_standard_f(req.fixed_rows.clone(), req.off_lo.clone(), lo, hi, legal, 300)  # untagged, equal by value
    bad = req.fixed_rows.clone()
    bad[0, 1, 5] += 1
    with pytest.raises(ValueError, match="selection rule"):
        check_standard_f(bad, req.off_lo, lo, hi, legal, 300)
    with pytest.raises(ValueError, match="selection rule"):
        check_standard_f(req.fixed_rows.clone(), req.off_lo.clone() + 1, lo, hi, legal, 300)
    with pytest.raises(ValueError, match="selection rule"):                            # a different capacity
        check_standard_f(req.fixed_rows.clone(), req.off_lo.clone(), lo, hi, legal, 301)
    assert torch.equal(req.fixed_rows[1, 2], req.fixed_positions[1, 2] + (1 * 3 + 2) * 300)


@pytest.mark.parametrize("kind", ["dynamic", "static"])
def test_native_runner_rolls_back_either_cache_kind(kind):
    """NativeRunner.rollback on transformers' growing (dynamic) and preallocated (static) caches: after rolling back
    to 40 tokens, the replayed steps equal the first pass, and the cache reports 40 + replayed tokens."""
    from transformers import DynamicCache, StaticCache
    from attention_lab.qwen_wrap import NativeRunner
    m = tiny_qwen3(seed=3)
    ids = torch.randint(0, 256, (1, 52), generator=torch.Generator().manual_seed(4))
    cache = DynamicCache(config=m.config) if kind == "dynamic" else StaticCache(config=m.config, max_cache_len=64)
    with torch.inference_mode():
        ref = m(ids).logits
        run = NativeRunner(m, cache, 64)
        run.prefill(ids[:, :40], 16)
        first = torch.cat([run.step(ids[:, i:i + 1]) for i in range(40, 52)], 1)
        torch.testing.assert_close(first, ref[:, 40:], rtol=1e-9, atol=1e-9)
        run.rollback(40)
        assert run.length == 40
        with pytest.raises(ValueError):
            run.rollback(41)
        again = torch.cat([run.step(ids[:, i:i + 1]) for i in range(40, 52)], 1)
        torch.testing.assert_close(again, first, rtol=0, atol=0)
        assert int(cache.get_seq_length()) == 52
