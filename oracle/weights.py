"""GroupedIndexer's seeded weights restated (src/attention_lab/indexer.py:38-45). Test infrastructure only.

A torch CPU generator seeded with `seed` draws wq [G, r, h*d] then wk [G, r, d] in float64, both scaled by
init_std; wq_t_scaled = (wq / sqrt(r)) transposed to [G, h*d, r]. Pinned by tests/golden/grouped_indexer.npz, which
tests/golden/make_golden.py wrote from the reference's own class.
"""
from __future__ import annotations

import math

import torch


def grouped_indexer_weights(groups: int, heads_per_group: int, head_dim: int, r: int = 32, seed: int = 0,
                            init_std: float = 0.02):
    gen = torch.Generator().manual_seed(int(seed))
    wq = torch.randn(groups, r, heads_per_group * head_dim, generator=gen, dtype=torch.float64) * init_std
    wk = torch.randn(groups, r, head_dim, generator=gen, dtype=torch.float64) * init_std
    wq_t_scaled = (wq / math.sqrt(r)).transpose(1, 2).contiguous()
    return wq.numpy(), wk.numpy(), wq_t_scaled.numpy()
