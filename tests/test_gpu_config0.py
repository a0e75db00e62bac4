"""The north_star's CPU-runnable case end to end on the GPU, against the oracle: one Qwen3-0.6B-shaped decode layer,
batch 1, L = 2048, 16 query heads over 8 KV heads, head_dim 128, bf16 K/V ~ N(0, 1); a lightning indexer of 4 heads,
r = 32, fp16 keys ~ N(0, 1/32), query ~ N(0, 1), head weights ~ U(0, 1); k = 64 positions (rho = 1/32). Outputs: fp32
scores, the top-64 indices, the sparse attention over them and the full attention.

Bars, written here: scores within 1e-5 of the float64 oracle relative to the largest |score|; the top-64 index list
bit-exact against the oracle's selection on the kernel's own fp32 scores (score order, ties to the lower index);
attention in fp32 within 5e-5 absolute and 1e-5 relative norm of the float64 read over the same rows (the bars of the
reference's attend tests, test_metal_attend.py:28-29), and the bf16 output within the north_star's bf16 bound.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from attention_lab import hip_attend, hip_score, hip_select
from oracle import bf16, exact

pytestmark = pytest.mark.gpu
f64 = bf16.values
B, G, h, d, L, NH, R, K_SEL = 1, 8, 2, 128, 2048, 4, 32, 64


def case(seed):
    gen = torch.Generator().manual_seed(seed)
    K = torch.randn(B, G, L, d, generator=gen).to(torch.bfloat16)
    V = torch.randn(B, G, L, d, generator=gen).to(torch.bfloat16)
    q = torch.randn(B, G, h, d, generator=gen).to(torch.bfloat16)
    keys = (torch.randn(B, 1, L, R, generator=gen) / R ** 0.5).to(torch.float16)     # one index key per position
    qi = torch.randn(B, 1, NH, R, generator=gen)
    w = torch.rand(B, 1, NH, generator=gen)
    return K, V, q, keys, qi, w


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_config0_layer_end_to_end(gpu, seed):
    K, V, q, keys, qi, w = case(seed)
    s = hip_score.score_lightning(keys.to(gpu), qi.to(gpu), w.to(gpu), 0, L, relu=True)       # [1, 1, L] fp32
    _, top = hip_select.topk(s.view(1, L), K_SEL, order="score")
    torch.cuda.synchronize()
    # scores
    want_s = exact.lightning_scores(f64(keys), f64(qi), f64(w), 0, L, relu=True)
    got_s = s.cpu().numpy().astype(np.float64)
    assert np.abs(got_s - want_s).max() <= 1e-5 * max(1.0, np.abs(want_s).max())
    # the top-64, on the kernel's own scores
    want_top = exact.topk(s.view(1, L).cpu().numpy(), K_SEL, order="score")
    assert np.array_equal(top.cpu().numpy(), want_top)
    # sparse attention over those rows (shared by every KV group) and the full read
    rows = top.view(1, 1, K_SEL).expand(B, G, K_SEL).to(torch.int32).contiguous()
    Kd, Vd, qd = K.to(gpu), V.to(gpu), q.to(gpu)
    sp32 = hip_attend.attend(qd, Kd, Vd, rows, out_dtype=torch.float32)
    sp16 = hip_attend.attend(qd, Kd, Vd, rows, out_dtype=torch.bfloat16)
    full32 = hip_attend.dense_decode(qd, Kd, Vd, L, out_dtype=torch.float32)
    torch.cuda.synchronize()
    rows_np = np.broadcast_to(want_top.reshape(1, 1, K_SEL), (B, G, K_SEL))
    want_sp = exact.subset_attention(f64(q), f64(K), f64(V), rows_np)
    want_full = exact.dense_attention(f64(q), f64(K), f64(V), L)
    for got, want, what in ((sp32, want_sp, "sparse"), (full32, want_full, "full")):
        diff = np.abs(got.cpu().numpy().astype(np.float64) - want)
        assert diff.max() <= 5e-5, f"{what}: max {diff.max():.3e}"
        assert np.linalg.norm(diff) <= 1e-5 * np.linalg.norm(want), f"{what}: relative norm"
    d16 = np.abs(f64(sp16) - want_sp)
    assert d16.max() <= 2e-2 and d16.mean() <= 2e-3
