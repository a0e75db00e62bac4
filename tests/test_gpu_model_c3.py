"""BASELINE configs[3] on the GPU through the wrapper: a random-init Qwen3-1.7B-shaped model (28 layers, hidden 2048,
16q/8kv, head_dim 128, FFN 6144, vocab 151936, rope theta 1e6, bf16 weights ~ N(0, 0.02)), an 8192-token uniform
prompt, then greedy decode steps (reference tests/test_qwen_wrapper.py:150-173 and :455-480, bench/model_numerics.py:
54-146).

Checks, with the tolerances stated here:
  * the full read (A, the dense decode kernel, bf16) against the unwrapped model run in float32 with transformers'
    eager attention over the same tokens: per-step logits within relative norm 0.08 and mean KL 5e-3 (bf16 weights and
    activations through 28 layers; this build measured 0.038 and 5.8e-4 over 128 steps);
  * the sparse read with k0 = capacity (every candidate selected, the reference's sparse == dense invariant) in both
    row orders (position order, and score order, the wrapper's default): against the same float32 reference no worse
    than twice the full read's own deviation (the reference's pre-registered bf16 rule, configs/mac_gate1b.json
    `revised_bfloat16_rule`, factor 2), and against the full read within relative norm 0.06.
The float32 reference runs last, after the bf16 model is converted, and never in bfloat16 (bf16 batched products with a
transposed operand are avoided on these boxes).
"""
from __future__ import annotations

import pytest
import torch

transformers = pytest.importorskip("transformers")

pytestmark = pytest.mark.gpu
PROMPT, STEPS = 8192, 4
A_REL, A_KL = 0.08, 5e-3
FACTOR, D_VS_A_REL = 2.0, 0.06


def qwen3_1p7b(dev, seed=0):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=151936, hidden_size=2048, intermediate_size=6144, num_hidden_layers=28,
                      num_attention_heads=16, num_key_value_heads=8, head_dim=128, max_position_embeddings=40960,
                      rope_theta=1_000_000.0, rms_norm_eps=1e-6, tie_word_embeddings=True, initializer_range=0.02,
                      attn_implementation="sdpa")
    torch.manual_seed(seed)
    with torch.device(dev):
        model = Qwen3ForCausalLM(cfg)
    model = model.to(torch.bfloat16).eval()
    for p in model.parameters():
        p.requires_grad_(False)
    return model


def deviation(a, b):
    """a against b, [n, V] logits: relative norm of the difference and the mean KL(b || a)."""
    a, b = a.float(), b.float()
    lp, lq = torch.log_softmax(b, -1), torch.log_softmax(a, -1)
    return float((a - b).norm() / b.norm()), float((lp.exp() * (lp - lq)).sum(-1).mean())


def test_configs3_qwen3_1p7b_8192_prompt(gpu):
    from attention_lab.qwen_wrap import LabRunner, make_state, unwrap_model, wrap_model
    model = qwen3_1p7b(gpu)
    holder = wrap_model(model)
    gen = torch.Generator(device=gpu)
    gen.manual_seed(0)
    prompt = torch.randint(0, model.config.vocab_size, (1, PROMPT), device=gpu, generator=gen)
    cap = PROMPT + STEPS + 1
    with torch.inference_mode():
        full = LabRunner(model, holder, make_state(model, cap, "full"))
        last = full.prefill(prompt, 2048)[:, -1].float()
        tokens, logits_a = [], [last]
        tok = last.argmax(-1, keepdim=True)
        for _ in range(STEPS):
            tokens.append(tok)
            lg = full.step(tok)[:, -1].float()
            logits_a.append(lg)
            tok = lg.argmax(-1, keepdim=True)
        logits_a = torch.cat(logits_a)                          # prompt end + STEPS steps
        del full
        print(f"[c3] full read: {STEPS} steps after an {PROMPT}-token prefill", flush=True)
        sparse = {}
        for order, canonical in (("position", True), ("score", False)):
            st = make_state(model, cap, "sparse", canonical_order=canonical)
            run = LabRunner(model, holder, st)
            first = run.prefill(prompt, 2048)[:, -1].float()
            st.begin_request(None, k0=cap)                     # every candidate on every step
            outs = [first]
            for i in range(STEPS):
                outs.append(run.step(tokens[i])[:, -1].float())
                assert st.plan.selected_count == st.plan.legal_length
            sparse[order] = torch.cat(outs)
            del run, st
            print(f"[c3] sparse read, k0 = capacity, {order} order", flush=True)
        unwrap_model(model)
        ref_model = model.float()
        ref_model.config._attn_implementation = "eager"
        ids = torch.cat([prompt] + tokens, dim=1)
        ref = ref_model(input_ids=ids, use_cache=False, logits_to_keep=STEPS + 1).logits[0].float()
        print("[c3] float32 eager reference done", flush=True)
    a_rel, a_kl = deviation(logits_a, ref)
    assert torch.isfinite(logits_a).all()
    assert a_rel <= A_REL and a_kl <= A_KL, f"full read vs float32: rel {a_rel:.3e} kl {a_kl:.3e}"
    for order, d in sparse.items():
        assert torch.isfinite(d).all()
        d_rel, d_kl = deviation(d, ref)
        assert d_rel <= FACTOR * a_rel, f"{order}: sparse (k0 = capacity) vs float32 rel {d_rel:.3e} > 2 x {a_rel:.3e}"
        assert d_kl <= FACTOR * a_kl + 1e-6, f"{order}: sparse vs float32 kl {d_kl:.3e} > 2 x {a_kl:.3e}"
        da_rel, _ = deviation(d, logits_a)
        assert da_rel <= D_VS_A_REL, f"{order}: sparse (k0 = capacity) vs full read rel {da_rel:.3e}"
        print(f"[c3] {order}: vs float32 rel {d_rel:.3e} kl {d_kl:.3e}; vs full read rel {da_rel:.3e} "
              f"(full read vs float32 rel {a_rel:.3e} kl {a_kl:.3e})", flush=True)


def test_configs3_partial_read_at_rho_1_32_touches_only_its_rows(gpu):
    """configs[3] at its real budget: after the 8192-token prompt, one decode step at rho = 1/32 (k0 = 256 of 8125
    candidates) in both row orders, with every layer's row list recorded. Each list holds S = 68 + k unique positions
    inside the legal range, F among them ([0, 4) and the last 64), the candidates inside [lo, hi); position order is
    strictly ascending, score order puts F first. Then every K/V row the step did not select is poisoned with NaN in
    every layer (and every unwritten slot), the step is replayed after a rollback, and its logits are bit-identical to
    the clean step while the dense read of the same cache turns non-finite (reference
    tests/test_qwen_wrapper.py:150-208 at model scale)."""
    from attention_lab.decode import dense_decode_step
    from attention_lab.qwen_wrap import LabRunner, make_state, unwrap_model, wrap_model
    from attention_lab.selection import fixed_budget
    model = qwen3_1p7b(gpu, seed=1)
    holder = wrap_model(model)
    gen = torch.Generator(device=gpu)
    gen.manual_seed(1)
    prompt = torch.randint(0, model.config.vocab_size, (1, PROMPT), device=gpu, generator=gen)
    tok = torch.randint(0, model.config.vocab_size, (1, 1), device=gpu, generator=gen)
    cap = PROMPT + 8
    L = PROMPT + 1
    lo, hi = 4, L - 64
    with torch.inference_mode():
        for canonical in (True, False):
            st = make_state(model, cap, "sparse", canonical_order=canonical)
            run = LabRunner(model, holder, st)
            run.prefill(prompt, 2048)
            assert st.begin_request(1 / 32) == fixed_budget(L, 1 / 32)
            st.record_selection = True
            clean = run.step(tok)
            plan = st.plan
            k, S = plan.k, plan.selected_count
            assert (plan.legal_length, plan.lo, plan.hi, S) == (L, lo, hi, 68 + k) and k == st.k0 < hi - lo
            cache = st.cache
            G, C = cache.groups, cache.slots
            fixed = torch.cat([torch.arange(4, device=gpu), torch.arange(L - 64, L, device=gpu)])
            keep_all = []
            for l in range(cache.layers):
                rows = (st.last_rows[l].view(1, G, S) - cache.offsets)[0]
                assert int(rows.min()) >= 0 and int(rows.max()) < L, f"layer {l}: a row outside the legal range"
                srt = rows.sort(dim=-1).values
                assert bool((srt[:, 1:] > srt[:, :-1]).all()), f"layer {l}: repeated rows"
                assert bool(torch.isin(fixed, rows).all()), f"layer {l}: F missing from the row list"
                if canonical:
                    assert torch.equal(rows, srt), f"layer {l}: position order not ascending"
                else:
                    assert torch.equal(rows[:, :68], fixed.expand(G, 68)), f"layer {l}: score order must start with F"
                    cand = rows[:, 68:]
                    assert bool(((cand >= lo) & (cand < hi)).all()), f"layer {l}: a candidate outside [lo, hi)"
                keep = torch.zeros(G, C, dtype=torch.bool, device=gpu)
                keep.scatter_(1, rows.long(), True)
                keep_all.append(keep)
            for l in range(cache.layers):
                drop = ~keep_all[l]
                cache.k[l][0][drop] = float("nan")
                cache.v[l][0][drop] = float("nan")
            run.rollback(PROMPT)
            poisoned = run.step(tok)
            assert torch.isfinite(poisoned).all(), "the sparse read touched a row it did not select"
            assert torch.equal(poisoned, clean), "poisoning unselected rows changed the sparse step's logits"
            q = torch.randn(1, G, 2, 1, 128, device=gpu, generator=gen).to(torch.bfloat16)
            dense = dense_decode_step(q, cache.k[0], cache.v[0], L)
            assert not bool(torch.isfinite(dense.float()).all()), "the dense read must see the poison"
            print(f"[c3] rho = 1/32, {'position' if canonical else 'score'} order: k = {k}, S = {S}, 28 layers, "
                  "poisoned replay bit-identical", flush=True)
            del run, st, cache, keep_all
        unwrap_model(model)
