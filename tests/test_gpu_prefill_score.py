"""Batched (prefill) lightning score on the matrix cores against the oracle and against the one-query kernel.

Tolerances, written here: fp32 scores against the float64 oracle on the same fp16/bf16 keys and fp32 queries, max |d|
<= 1e-5 * max(1, max |ref|) and relative norm <= 1e-5 (north_star asks 1e-3 relative); against the one-query kernel
(fp32 FMAs in another order) 2e-6 * max(1, max |score|). Entries past a query's causal bound must keep what `out`
held (the kernel does not write them).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from attention_lab import _native as nat
from attention_lab import hip_score
from oracle import bf16, exact

pytestmark = pytest.mark.gpu
TOL = {"atol_scale": 1e-5, "rel_norm": 1e-5, "vs_one_query": 2e-6}
f64 = bf16.values
SENTINEL = 12345.0


def inputs(B, KG, L, T, nh, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    keys = (torch.randn(B, KG, L, 32, generator=gen) / 32 ** 0.5).to(dtype)
    q = torch.randn(B, KG, T, nh, 32, generator=gen)
    w = torch.rand(B, KG, T, nh, generator=gen)
    return keys, q, w


def check(got, ref, what):
    got = f64(got)
    valid = ~np.isnan(ref)
    scale = max(1.0, float(np.abs(ref[valid]).max()))
    diff = float(np.abs(got[valid] - ref[valid]).max())
    rel = float(np.linalg.norm(got[valid] - ref[valid]) / np.linalg.norm(ref[valid]))
    assert diff <= TOL["atol_scale"] * scale, f"{what}: max abs diff {diff:.3e} (scale {scale:.2e})"
    assert rel <= TOL["rel_norm"], f"{what}: rel norm {rel:.3e}"
    untouched = got[~valid]
    assert np.all(untouched == SENTINEL), f"{what}: {np.count_nonzero(untouched != SENTINEL)} entries past the causal " \
                                          "bound were written"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("nh,relu", [(1, False), (2, True), (4, True), (8, False), (4, False)])
@pytest.mark.parametrize("q_pos0", [None, 2300, 40])
def test_matches_oracle(gpu, dtype, nh, relu, q_pos0):
    B, KG, L, T = 2, 3, 2500, 70
    lo, hi = 4, L - 64
    keys, q, w = inputs(B, KG, L, T, nh, dtype, seed=nh + 10 * (q_pos0 or 0))
    M = hi - lo
    out = torch.full((B, KG, T, (M + 3) // 4 * 4), SENTINEL, device=gpu)
    s = hip_score.score_lightning_batched(keys.to(gpu), q.to(gpu), w.to(gpu), lo, hi, q_pos0=q_pos0, relu=relu,
                                          out=out)
    torch.cuda.synchronize()
    ref = exact.lightning_scores_batched(f64(keys), f64(q), f64(w), lo, hi, q_pos0=q_pos0, relu=relu)
    check(s, ref, f"{dtype} nh={nh} relu={relu} q_pos0={q_pos0}")


@pytest.mark.parametrize("nh", [1, 4, 8])
def test_each_query_equals_the_one_query_kernel(gpu, nh):
    B, KG, L, T = 1, 2, 3000, 33
    keys, q, w = (x.to(gpu) for x in inputs(B, KG, L, T, nh, torch.float16, seed=7))
    lo, hi = 4, L
    s = hip_score.score_lightning_batched(keys, q, w, lo, hi)
    for t in (0, 1, 17, T - 1):
        one = hip_score.score_lightning(keys, q[:, :, t].contiguous(), w[:, :, t].contiguous(), lo, hi)
        torch.cuda.synchronize()
        scale = max(1.0, float(one.abs().max()))
        assert float((s[:, :, t] - one).abs().max()) <= TOL["vs_one_query"] * scale, f"query {t}"


def test_long_prefill_chunk_against_fp32_on_the_device(gpu):
    """A 512-query chunk at the end of a 32K context (causal), nh = 4, fp16 keys: scores against an fp32 matmul of the
    same operands on the device, on every written entry."""
    B, KG, L, T, nh = 1, 2, 32768, 512, 4
    gen = torch.Generator(device=gpu).manual_seed(3)
    keys = (torch.randn(B, KG, L, 32, generator=gen, device=gpu) / 32 ** 0.5).to(torch.float16)
    q = torch.randn(B, KG, T, nh, 32, generator=gen, device=gpu)
    w = torch.rand(B, KG, T, nh, generator=gen, device=gpu)
    p0 = L - T
    out = torch.full((B, KG, T, L), SENTINEL, device=gpu)
    s = hip_score.score_lightning_batched(keys, q, w, 0, L, q_pos0=p0, out=out)
    dots = torch.matmul(q.view(B, KG, T * nh, 32), keys.float().transpose(2, 3)).view(B, KG, T, nh, L)
    ref = (dots.clamp_min(0.0) * w.unsqueeze(-1)).sum(3)
    m = torch.arange(L, device=gpu).view(1, L)
    t = torch.arange(T, device=gpu).view(T, 1)
    valid = (m <= p0 + t).view(1, 1, T, L).expand_as(ref)
    torch.cuda.synchronize()
    scale = max(1.0, float(ref.abs().max()))
    assert float((s - ref).abs()[valid].max()) <= TOL["atol_scale"] * scale
    assert bool((s[~valid] == SENTINEL).all())


def test_empty_and_validation(gpu):
    keys, q, w = (x.to(gpu) for x in inputs(1, 1, 100, 4, 2, torch.float16, seed=1))
    assert hip_score.score_lightning_batched(keys, q, w, 10, 10).shape == (1, 1, 4, 0)
    z = hip_score.score_lightning_batched(keys, q[:, :, :0].contiguous(), w[:, :, :0].contiguous(), 0, 100)
    assert z.shape == (1, 1, 0, 100)
    with pytest.raises(ValueError):   # nh = 3
        hip_score.score_lightning_batched(keys, torch.zeros(1, 1, 4, 3, 32, device=gpu),
                                          torch.zeros(1, 1, 4, 3, device=gpu))
    with pytest.raises(ValueError):   # out row not a multiple of 4
        hip_score.score_lightning_batched(keys, q, w, 0, 99, out=torch.empty(1, 1, 4, 99, device=gpu))
    with pytest.raises(ValueError):
        hip_score.score_lightning_batched(keys, q, w, 0, 100, q_pos0=-2)
    with pytest.raises(ValueError):
        hip_score.score_lightning_batched(keys, q, w, 0, 101)
    out = torch.empty(4 * 100 + 4, device=gpu)
    with pytest.raises(ValueError):   # the C ABI's own stride check
        nat.call("attnlab_score_lightning_batched", keys.data_ptr(), nat.DT_F16, q.data_ptr(), w.data_ptr(),
                 out.data_ptr(), 101, 1, 1, 100, 32, 2, 4, 0, 100, -1, 1, nat.stream_of(gpu))
