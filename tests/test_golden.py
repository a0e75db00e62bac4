"""GroupedIndexer weights against the golden vectors written from the reference's own class (tests/golden/)."""
from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np
import pytest
import torch

from attention_lab.indexer import GroupedIndexer
from oracle.weights import grouped_indexer_weights

GOLDEN = np.load(Path(__file__).resolve().parent / "golden" / "grouped_indexer.npz", allow_pickle=False)


def _cases(prefix):
    out = set()
    for name in GOLDEN.files:
        if name.startswith(prefix):
            parts = name.split("_")
            out.add(tuple(int(x) for x in parts[1:6]))
    return sorted(out)


def _digest(a):
    return hashlib.sha256(np.ascontiguousarray(a, dtype=np.float64).tobytes()).hexdigest()


@pytest.mark.parametrize("G,h,d,r,seed", _cases("small"))
def test_small_weights_bit_exact(G, h, d, r, seed):
    tag = f"small_{G}_{h}_{d}_{r}_{seed}"
    idx = GroupedIndexer(G, h, d, r, dtype=torch.float64, seed=seed)
    o_wq, o_wk, o_wqt = grouped_indexer_weights(G, h, d, r, seed)
    for name, prod, orc in (("wq", idx.wq, o_wq), ("wk", idx.wk, o_wk), ("wq_t_scaled", idx.wq_t_scaled, o_wqt)):
        want = GOLDEN[f"{tag}_{name}"]
        assert np.array_equal(prod.numpy(), want), f"product {name} differs from the reference"
        assert np.array_equal(orc, want), f"oracle {name} differs from the reference"


@pytest.mark.parametrize("G,h,d,r,seed", _cases("big"))
def test_qwen_shaped_weights_digest(G, h, d, r, seed):
    tag = f"big_{G}_{h}_{d}_{r}_{seed}"
    idx = GroupedIndexer(G, h, d, r, dtype=torch.float64, seed=seed)
    for name in ("wq", "wk", "wq_t_scaled"):
        a = getattr(idx, name).numpy()
        assert np.array_equal(a.reshape(-1)[:16], GOLDEN[f"{tag}_{name}_head"])
        assert _digest(a) == str(GOLDEN[f"{tag}_{name}_sha256"]), f"{name} digest differs from the reference"


def test_bf16_weights_are_the_rounded_float64_draws():
    idx64 = GroupedIndexer(8, 2, 128, 32, dtype=torch.float64, seed=0)
    idx16 = GroupedIndexer(8, 2, 128, 32, dtype=torch.bfloat16, seed=0)
    assert torch.equal(idx16.wk, idx64.wk.to(torch.bfloat16))
    assert torch.equal(idx16.wq_t_scaled, idx64.wq_t_scaled.to(torch.bfloat16))
