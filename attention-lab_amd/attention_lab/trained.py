"""Frozen trained index banks: hash-verified float32 (Wq, Wk) per layer and the float32 index table they score.

Mirrors src/attention_lab/trained.py:11-81: `FrozenIndexer` (float32 weights, 1/sqrt(r) folded into wq_t_scaled,
a version signature that catches in-place edits), `FrozenBank.guard` (the checks a LabRunner makes before any cache
write), `load_bank` (metadata identity, complete layer set, paths inside the run, SHA-256 per file, geometry and
finiteness, `allow_pickle=False`) and `make_trained_state` (a float32 index cache and canonical row order). The
messages are the reference's, so callers matching on them keep working. On this build the float32 table is scored by
the fp32 kernels of libattnlab.so (attnlab_score_grouped_f32, attnlab_project_keys_f32,
attnlab_sparse_decode_step_f32); the model's own K/V cache stays bfloat16.
"""
from __future__ import annotations

import hashlib
import json
import math
from pathlib import Path

import numpy as np
import torch

__all__ = ["FrozenIndexer", "FrozenBank", "load_bank", "make_trained_state", "bank_id"]


def bank_id(metadata: dict) -> str:
    """SHA-256 of the metadata without its own `bank_id`, keys sorted (trained.py:54-56)."""
    unsigned = {k: v for k, v in metadata.items() if k != "bank_id"}
    return hashlib.sha256(json.dumps(unsigned, sort_keys=True).encode()).hexdigest()


class FrozenIndexer:
    """One layer's learned index (trained.py:11-27). wq [G, r, h*d] and wk [G, r, d] must be float32 arrays."""

    def __init__(self, wq: np.ndarray, wk: np.ndarray, *, identity: str, device):
        if wq.dtype != np.float32 or wk.dtype != np.float32:
            raise ValueError("frozen index parameters must be float32")
        self.wq = torch.from_numpy(np.array(wq, copy=True)).to(device).detach()
        self.wk = torch.from_numpy(np.array(wk, copy=True)).to(device).detach()
        self.r = int(self.wk.shape[1])
        self.wq_t_scaled = (self.wq / math.sqrt(self.r)).transpose(1, 2).contiguous()
        self.identity = identity
        self._versions = self.signature()

    def signature(self):
        """Object ids and in-place version counters of the three parameter tensors."""
        return tuple((id(t), t._version) for t in (self.wq, self.wk, self.wq_t_scaled))

    def verify(self):
        if self.signature() != self._versions:
            raise RuntimeError("frozen index parameters changed; rebuild bank and prefix cache")


class FrozenBank:
    """The layer indexes of one bank plus the identity bound into every cache it fills (trained.py:30-48)."""

    def __init__(self, indexes, *, identity: str):
        self.indexes = list(indexes)
        self.identity = identity
        self._objects = tuple(id(x) for x in self.indexes)

    def guard(self, state):
        """LabState.cache_guard: run before a forward writes anything to the cache."""
        if tuple(id(x) for x in state.indexers) != self._objects:
            raise RuntimeError("state index bank changed")
        cache = state.cache
        for index in self.indexes:
            index.verify()
            if index.wk.device != cache.device:
                raise RuntimeError("index/cache devices differ")
        if not cache.has_index or cache.index_dtype != torch.float32:
            raise RuntimeError("bank requires a float32 index cache")
        if cache.valid_length and getattr(cache, "index_identity", None) != self.identity:
            raise RuntimeError("prefix index cache belongs to different parameter identity")
        cache.index_identity = self.identity


def load_bank(run_dir, metadata: dict, geometry, *, device, initial: bool = False) -> FrozenBank:
    """Verify every file, then load the "final" (or "initial") parameters of each layer (trained.py:51-75).

    metadata: {"bank_id", "r", "layers": [{"layer_index", "<role>_file", "<role>_sha256"}, ...], ...};
    geometry: anything with layers, groups, heads_per_group and head_dim (qwen_wrap.geometry_of).
    """
    root = Path(run_dir).resolve()
    if bank_id(metadata) != metadata["bank_id"]:
        raise ValueError("bank metadata identity mismatch")
    entries = metadata["layers"]
    if len(entries) != geometry.layers or {e["layer_index"] for e in entries} != set(range(geometry.layers)):
        raise ValueError("incomplete index bank")
    r = metadata["r"]
    role = "initial" if initial else "final"
    want_q = (geometry.groups, r, geometry.heads_per_group * geometry.head_dim)
    want_k = (geometry.groups, r, geometry.head_dim)
    indexes = []
    for entry in sorted(entries, key=lambda e: e["layer_index"]):
        path = (root / entry[role + "_file"]).resolve()
        if not path.is_relative_to(root):
            raise ValueError("parameter path outside run")
        blob = path.read_bytes()
        identity = hashlib.sha256(blob).hexdigest()
        if identity != entry[role + "_sha256"]:
            raise ValueError("parameter file hash mismatch")
        with np.load(path, allow_pickle=False) as f:
            wq, wk = f["wq"], f["wk"]
        if wq.shape != want_q or wk.shape != want_k:
            raise ValueError("index/model geometry differs")
        if not np.isfinite(wq).all() or not np.isfinite(wk).all():
            raise ValueError("nonfinite parameters")
        indexes.append(FrozenIndexer(wq, wk, identity=identity, device=device))
    identity = hashlib.sha256(json.dumps({"bank_id": metadata["bank_id"], "role": role,
                                          "files": [x.identity for x in indexes], "r": r, "dtype": "float32"},
                                         sort_keys=True).encode()).hexdigest()
    return FrozenBank(indexes, identity=identity)


def make_trained_state(model, capacity: int, bank: FrozenBank, *, sparse_layers=None, mode: str = "sparse"):
    """A LabState over a float32 index cache, guarded by the bank, rows in ascending order (trained.py:78-81)."""
    from .qwen_wrap import LabState, make_cache
    cache = make_cache(model, capacity, with_index=True, index_dim=bank.indexes[0].r, index_dtype=torch.float32)
    return LabState(cache, bank.indexes, mode=mode, selector="index", sparse_layers=sparse_layers,
                    cache_guard=bank.guard, canonical_order=True)
