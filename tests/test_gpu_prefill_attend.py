"""Causal prefill read on the matrix cores (attnlab_prefill_attend) against the float64 oracle and an fp32 reference.

The reference's legality rule (reference.py:41-48): key j is legal for query t iff j <= its position and
j < valid_length. Tolerances, written here: the north_star's bf16 attention bar, max |d| <= 2e-2 and mean |d| <= 2e-3
against the float64 oracle on the same bf16 inputs.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from attention_lab import _native as nat
from attention_lab import hip_attend
from attention_lab.full import full_attention
from oracle import bf16, exact

pytestmark = pytest.mark.gpu
TOL = {"max_abs": 2e-2, "mean_abs": 2e-3}
f64 = bf16.values


def inputs(gpu, B, G, h, T, C, seed):
    gen = torch.Generator().manual_seed(seed)
    K = torch.randn(B, G, C, 128, generator=gen).to(torch.bfloat16)
    V = torch.randn(B, G, C, 128, generator=gen).to(torch.bfloat16)
    q = torch.randn(B, G, h, T, 128, generator=gen).to(torch.bfloat16)
    return K.to(gpu), V.to(gpu), q.to(gpu)


def check(out, want, what):
    diff = np.abs(f64(out) - want)
    assert float(diff.max()) <= TOL["max_abs"], f"{what}: max abs {diff.max():.3e}"
    assert float(diff.mean()) <= TOL["mean_abs"], f"{what}: mean abs {diff.mean():.3e}"


@pytest.mark.parametrize("h", [1, 2, 4, 8])
@pytest.mark.parametrize("T,p0,cut", [(1, 0, 0), (5, 0, 0), (64, 37, 0), (130, 0, 0), (130, 200, 40), (300, 61, 7)])
def test_matches_the_oracle(gpu, h, T, p0, cut):
    """Chunks at position 0 and later, chunk lengths that are and are not multiples of a workgroup's 128 / h queries,
    and a valid_length that cuts the chunk's last queries' reads short (`cut` rows)."""
    B, G = 2, 3
    legal = p0 + T - cut
    C = p0 + T + 11
    K, V, q = inputs(gpu, B, G, h, T, C, seed=h * 1000 + T + p0)
    out = hip_attend.prefill_attend(q, K, V, p0, legal)
    torch.cuda.synchronize()
    want = exact.causal_attention(f64(q), f64(K), f64(V), legal, list(range(p0, p0 + T)))
    check(out, want, f"h={h} T={T} p0={p0} legal={legal}")


@pytest.mark.parametrize("scale", [0.0, -0.09, 0.2])
def test_scales_other_than_the_default(gpu, scale):
    """A zero scale (uniform weights over the legal keys), a negative one (the kernel flips the query's sign and uses
    |scale|) and a larger positive one, against the float64 oracle with the same scale; chunk edges and a cut."""
    B, G, h, T, p0, cut = 2, 2, 4, 130, 61, 7
    legal = p0 + T - cut
    C = p0 + T + 11
    K, V, q = inputs(gpu, B, G, h, T, C, seed=77)
    out = hip_attend.prefill_attend(q, K, V, p0, legal, scale=scale)
    torch.cuda.synchronize()
    want = exact.causal_attention(f64(q), f64(K), f64(V), legal, list(range(p0, p0 + T)), scale=scale)
    check(out, want, f"scale={scale}")


def test_rows_past_valid_length_are_never_read(gpu):
    B, G, h, T, p0 = 1, 2, 2, 96, 40
    C = 200
    legal = p0 + T
    K, V, q = inputs(gpu, B, G, h, T, C, seed=5)
    ref = hip_attend.prefill_attend(q, K, V, p0, legal)
    K[:, :, legal:] = float("nan")
    V[:, :, legal:] = float("nan")
    out = hip_attend.prefill_attend(q, K, V, p0, legal)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all())
    assert torch.equal(out, ref)


def test_long_chunk_against_fp32_on_the_device(gpu):
    """2048 queries after 1000 cached positions (8 groups, 2 heads): every output against an fp32 masked softmax of
    the same bf16 operands, computed on the device in float32."""
    B, G, h, T, p0 = 1, 8, 2, 2048, 1000
    legal = p0 + T
    C = legal + 64
    gen = torch.Generator(device=gpu).manual_seed(11)
    K = torch.randn(B, G, C, 128, generator=gen, device=gpu).to(torch.bfloat16)
    V = torch.randn(B, G, C, 128, generator=gen, device=gpu).to(torch.bfloat16)
    q = torch.randn(B, G, h, T, 128, generator=gen, device=gpu).to(torch.bfloat16)
    out = hip_attend.prefill_attend(q, K, V, p0, legal)
    Kf, Vf = K[:, :, :legal].float().contiguous(), V[:, :, :legal].float().contiguous()
    s = torch.matmul(q.float().reshape(B, G, h * T, 128), Kf.transpose(2, 3).contiguous()) / math.sqrt(128)
    s = s.view(B, G, h, T, legal)
    pos = torch.arange(p0, p0 + T, device=gpu).view(T, 1)
    s = s.masked_fill(torch.arange(legal, device=gpu).view(1, legal) > pos, float("-inf"))
    want = torch.matmul(torch.softmax(s, -1).reshape(B, G, h * T, legal), Vf).view(B, G, h, T, 128)
    torch.cuda.synchronize()
    diff = (out.float() - want).abs()
    assert float(diff.max()) <= TOL["max_abs"] and float(diff.mean()) <= TOL["mean_abs"]


def test_full_attention_takes_the_prefill_kernel_for_consecutive_positions(gpu):
    B, G, h, T = 1, 2, 2, 70
    K, V, q = inputs(gpu, B, G, h, T, 150, seed=9)
    out = full_attention(q, K, V, valid_length=120)            # positions 50 .. 119
    direct = hip_attend.prefill_attend(q, K, V, 50, 120)
    torch.cuda.synchronize()
    assert torch.equal(out, direct)


def test_validation(gpu):
    K, V, q = inputs(gpu, 1, 1, 2, 4, 16, seed=1)
    with pytest.raises(ValueError):
        hip_attend.prefill_attend(q, K, V, 0, 17)                 # valid_length > capacity
    with pytest.raises(ValueError):
        hip_attend.prefill_attend(q, K, V, -1, 4)
    with pytest.raises(ValueError):
        hip_attend.prefill_attend(torch.zeros(1, 1, 3, 4, 128, dtype=torch.bfloat16, device=gpu), K, V, 0, 4)   # h=3
    out = torch.empty(1, 1, 2, 4, 128, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):   # the C ABI's own check (d must be 128)
        nat.call("attnlab_prefill_attend", q.data_ptr(), K.data_ptr(), V.data_ptr(), 16 * 128, 128, out.data_ptr(), 1,
                 1, 2, 4, 64, 0, 4, 16, 0.1, nat.stream_of(gpu))


@pytest.mark.parametrize("h", [1, 2, 8])
@pytest.mark.parametrize("splits", [2, 3, 4, 8])
@pytest.mark.parametrize("T,p0,cut", [(130, 1500, 9), (64, 0, 0), (300, 700, 0)])
def test_key_splits_match_the_oracle(gpu, h, splits, T, p0, cut):
    """The key-split read (attnlab_prefill_attend_split) against the float64 oracle: a chunk after a long history with a
    cut, a chunk at position 0 (the later splits of its early tiles hold no visible key) and a chunk whose split
    boundaries fall inside its tiles' visible ranges, at 128, 64 and 16 queries per tile (h = 1, 2, 8)."""
    B, G = 1, 2
    legal = p0 + T - cut
    C = p0 + T + 5
    K, V, q = inputs(gpu, B, G, h, T, C, seed=splits * 100 + T + h)
    out = hip_attend.prefill_attend(q, K, V, p0, legal, splits=splits)
    torch.cuda.synchronize()
    want = exact.causal_attention(f64(q), f64(K), f64(V), legal, list(range(p0, p0 + T)))
    check(out, want, f"splits={splits} T={T} p0={p0} legal={legal}")


def test_key_splits_against_the_unsplit_read_and_the_rule(gpu):
    """A 1K chunk after 7K cached positions at B=1, G=8, h=2 takes four splits by the rule; the merged output equals
    the one-pass read up to the summation order (within two bf16 ulps of 1 here), and rows past valid_length stay
    unread."""
    B, G, h, T, p0 = 1, 8, 2, 1024, 7168
    legal, C = p0 + T, p0 + T + 64
    assert hip_attend.prefill_splits(B, G, h, T, p0, legal) == 4
    assert hip_attend.prefill_splits(1, 8, 2, 8192, 0, 8192) == 1          # 1024 tiles: one per tile
    gen = torch.Generator(device=gpu).manual_seed(3)
    K = torch.randn(B, G, C, 128, generator=gen, device=gpu).to(torch.bfloat16)
    V = torch.randn(B, G, C, 128, generator=gen, device=gpu).to(torch.bfloat16)
    q = torch.randn(B, G, h, T, 128, generator=gen, device=gpu).to(torch.bfloat16)
    one = hip_attend.prefill_attend(q, K, V, p0, legal, splits=1)
    split = hip_attend.prefill_attend(q, K, V, p0, legal)
    K[:, :, legal:] = float("nan")
    V[:, :, legal:] = float("nan")
    again = hip_attend.prefill_attend(q, K, V, p0, legal)
    torch.cuda.synchronize()
    assert float((one.float() - split.float()).abs().max()) <= 2 ** -6
    assert torch.equal(again, split)


def test_key_split_validation(gpu):
    K, V, q = inputs(gpu, 1, 1, 2, 4, 16, seed=2)
    with pytest.raises(ValueError):
        hip_attend.prefill_attend(q, K, V, 0, 16, splits=17)
    out = torch.empty_like(q)
    need = nat.lib().attnlab_prefill_part_bytes(1, 1, 2, 4, 2)
    assert need == 1 * 1 * 2 * 4 * 2 * 132 * 4
    part = torch.empty(need // 4 - 1, dtype=torch.float32, device=gpu)
    with pytest.raises(ValueError):   # a part buffer one float short
        nat.call("attnlab_prefill_attend_split", q.data_ptr(), K.data_ptr(), V.data_ptr(), 16 * 128, 128,
                 out.data_ptr(), 1, 1, 2, 4, 128, 0, 16, 16, 0.1, 2, part.data_ptr(), (need // 4 - 1) * 4,
                 nat.stream_of(gpu))
