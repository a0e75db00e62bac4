"""Write tests/golden/grouped_indexer.npz from the reference's own GroupedIndexer (run in the build container only).

GroupedIndexer's weights come from a seeded torch generator (src/attention_lab/indexer.py:38-45); no closed form or
known answer in the reference's tests pins those draws, so this script imports the reference class once and records
its weights as vectors. Small shapes are stored whole (float64); the Qwen3-shaped ones as SHA-256 digests of the
float64 bytes plus a few leading values. Usage: python tests/golden/make_golden.py /root/reference
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "grouped_indexer.npz"
SMALL = [(2, 2, 16, 32, s) for s in (0, 1, 2)] + [(2, 4, 16, 8, 7)]
BIG = [(8, 2, 128, 32, 0), (8, 4, 128, 32, 0), (8, 2, 128, 32, 1001), (8, 2, 16, 32, 1000)]


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, dtype=np.float64).tobytes()).hexdigest()


def main(ref_root: str) -> None:
    sys.path.insert(0, str(Path(ref_root) / "src"))
    import torch
    from attention_lab.indexer import GroupedIndexer

    data = {}
    for G, h, d, r, seed in SMALL:
        idx = GroupedIndexer(G, h, d, r, dtype=torch.float64, seed=seed)
        tag = f"small_{G}_{h}_{d}_{r}_{seed}"
        data[tag + "_wq"] = idx.wq.numpy()
        data[tag + "_wk"] = idx.wk.numpy()
        data[tag + "_wq_t_scaled"] = idx.wq_t_scaled.numpy()
    for G, h, d, r, seed in BIG:
        idx = GroupedIndexer(G, h, d, r, dtype=torch.float64, seed=seed)
        tag = f"big_{G}_{h}_{d}_{r}_{seed}"
        for name in ("wq", "wk", "wq_t_scaled"):
            a = getattr(idx, name).numpy()
            data[f"{tag}_{name}_sha256"] = np.array(digest(a))
            data[f"{tag}_{name}_head"] = a.reshape(-1)[:16].copy()
    np.savez(OUT, **data)
    print(f"wrote {OUT} ({len(data)} arrays)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
