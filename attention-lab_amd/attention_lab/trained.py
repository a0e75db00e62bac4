"""Frozen trained index banks: per-layer float32 (Wq, Wk) loaded from hash-verified files, and the float32 index cache
they score (counterpart of src/attention_lab/trained.py:11-81).

Kept as the reference has them, because existing banks and their callers depend on them: the metadata identity
(SHA-256 of the key-sorted JSON without `bank_id`), the per-file SHA-256 named in the metadata, the bank identity
bound into every cache the bank fills, the role ("final" or "initial") as part of that identity, and the error
messages. How the checks are organised is this module's own: each layer file is verified by a `_LayerFile` before
anything is read from it, a `FrozenIndexer` watches its three parameter tensors for in-place edits, and the bank's
guard runs before a runner writes anything to the cache. On this build the float32 table is scored by the fp32
kernels (attnlab_score_grouped_f32, attnlab_project_keys_f32, attnlab_sparse_decode_step_f32); the model's K/V cache
stays bfloat16.
"""
from __future__ import annotations

import hashlib
import json
import math
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

__all__ = ["FrozenIndexer", "FrozenBank", "load_bank", "make_trained_state", "bank_id"]


def _sha256_json(obj) -> str:
    return hashlib.sha256(json.dumps(obj, sort_keys=True).encode()).hexdigest()


def bank_id(metadata: dict) -> str:
    """The metadata's identity: SHA-256 of its key-sorted JSON with the `bank_id` entry itself left out."""
    return _sha256_json({key: value for key, value in metadata.items() if key != "bank_id"})


class FrozenIndexer:
    """One layer's learned index: wq [G, r, h*d] and wk [G, r, d] as float32 tensors, wq_t_scaled = (wq / sqrt(r))^T.
    Any in-place change of the three tensors after construction makes verify() raise."""

    def __init__(self, wq: np.ndarray, wk: np.ndarray, *, identity: str, device):
        if wq.dtype != np.float32 or wk.dtype != np.float32:
            raise ValueError("frozen index parameters must be float32")
        self.wq = torch.tensor(wq, device=device)
        self.wk = torch.tensor(wk, device=device)
        self.r = int(self.wk.shape[1])
        self.wq_t_scaled = (self.wq / math.sqrt(self.r)).transpose(1, 2).contiguous()
        self.identity = identity
        self._watch = self._watched()

    def _watched(self):
        return tuple((t, t._version) for t in (self.wq, self.wk, self.wq_t_scaled))

    def signature(self):
        """(object id, in-place version) of wq, wk and wq_t_scaled."""
        return tuple((id(t), version) for t, version in self._watched())

    def verify(self):
        now = self._watched()
        if any(a is not b or va != vb for (a, va), (b, vb) in zip(now, self._watch)):
            raise RuntimeError("frozen index parameters changed; rebuild bank and prefix cache")


class FrozenBank:
    """A bank's layer indexes and the identity it binds into every cache it fills."""

    def __init__(self, indexes, *, identity: str):
        self.indexes = list(indexes)
        self.identity = identity
        self._members = tuple(map(id, self.indexes))

    def guard(self, state):
        """Run by LabRunner before a forward writes to the cache, then bind this bank's identity into the cache. The
        rules, each with the contract's message: the table is a float32 index table; the state holds exactly this
        bank's index objects; each is unedited and on the cache's device; a table that already holds keys was filled
        by this bank."""
        cache = state.cache
        for broken, message in self._rules(state, cache):
            if broken():
                raise RuntimeError(message)
        cache.index_identity = self.identity

    def _rules(self, state, cache):
        def edited():
            for index in self.indexes:
                index.verify()   # raises its own message
            return False
        return (
            (lambda: not cache.has_index or cache.index_dtype != torch.float32, "bank requires a float32 index cache"),
            (lambda: tuple(map(id, state.indexers or ())) != self._members, "state index bank changed"),
            (edited, ""),
            (lambda: any(index.wk.device != cache.device for index in self.indexes), "index/cache devices differ"),
            (lambda: bool(cache.valid_length) and getattr(cache, "index_identity", None) != self.identity,
             "prefix index cache belongs to different parameter identity"),
        )


@dataclass
class _LayerFile:
    """One layer's parameter file of a role, verified before use: inside the run directory, with the SHA-256 the
    metadata names, holding finite float32 arrays of the model's geometry (np.load with allow_pickle=False)."""
    root: Path
    entry: dict
    role: str

    def load(self, want_q: tuple, want_k: tuple):
        path = (self.root / self.entry[self.role + "_file"]).resolve()
        if not path.is_relative_to(self.root):
            raise ValueError("parameter path outside run")
        digest = hashlib.sha256(path.read_bytes()).hexdigest()
        if digest != self.entry[self.role + "_sha256"]:
            raise ValueError("parameter file hash mismatch")
        with np.load(path, allow_pickle=False) as arrays:
            wq, wk = arrays["wq"], arrays["wk"]
        if wq.shape != want_q or wk.shape != want_k:
            raise ValueError("index/model geometry differs")
        if not (np.isfinite(wq).all() and np.isfinite(wk).all()):
            raise ValueError("nonfinite parameters")
        return wq, wk, digest


def load_bank(run_dir, metadata: dict, geometry, *, device, initial: bool = False) -> FrozenBank:
    """Verify the metadata, the layer set and every file, then load the bank's "final" (or "initial") parameters.

    metadata: {"bank_id", "r", "layers": [{"layer_index", "<role>_file", "<role>_sha256"}, ...], ...};
    geometry: anything with layers, groups, heads_per_group and head_dim (qwen_wrap.geometry_of).
    """
    if bank_id(metadata) != metadata["bank_id"]:
        raise ValueError("bank metadata identity mismatch")
    entries = sorted(metadata["layers"], key=lambda e: e["layer_index"])
    if [e["layer_index"] for e in entries] != list(range(geometry.layers)):
        raise ValueError("incomplete index bank")
    r, role, root = metadata["r"], ("initial" if initial else "final"), Path(run_dir).resolve()
    want_q = (geometry.groups, r, geometry.heads_per_group * geometry.head_dim)
    want_k = (geometry.groups, r, geometry.head_dim)
    indexes = []
    for entry in entries:
        wq, wk, digest = _LayerFile(root, entry, role).load(want_q, want_k)
        indexes.append(FrozenIndexer(wq, wk, identity=digest, device=device))
    identity = _sha256_json({"bank_id": metadata["bank_id"], "role": role, "files": [x.identity for x in indexes],
                             "r": r, "dtype": "float32"})
    return FrozenBank(indexes, identity=identity)


def make_trained_state(model, capacity: int, bank: FrozenBank, *, sparse_layers=None, mode: str = "sparse"):
    """A LabState over a float32 index cache, guarded by the bank, with every row list in ascending order."""
    from .qwen_wrap import LabState, make_cache
    cache = make_cache(model, capacity, with_index=True, index_dim=bank.indexes[0].r, index_dtype=torch.float32)
    return LabState(cache, bank.indexes, mode=mode, selector="index", sparse_layers=sparse_layers,
                    cache_guard=bank.guard, canonical_order=True)
