"""Host contracts of frozen trained banks (reference tests/test_trained_inference.py:20-30 and :65-90, trained.py:11-81):
the float32-only indexer, its in-place-edit check, every verification load_bank makes before it trusts a file, and the
guard a runner calls before any cache write. No kernel runs here (device "cpu")."""
from __future__ import annotations

import hashlib
import json
import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from attention_lab.trained import FrozenBank, FrozenIndexer, bank_id, load_bank

GEO = SimpleNamespace(layers=2, groups=2, heads_per_group=2, head_dim=16)
R = 4


def write_bank(tmp_path, seed=100, geo=GEO, r=R):
    entries = []
    for layer in range(geo.layers):
        gen = np.random.default_rng(seed + layer)
        wq = (0.02 * gen.standard_normal((geo.groups, r, geo.heads_per_group * geo.head_dim))).astype(np.float32)
        wk = (0.02 * gen.standard_normal((geo.groups, r, geo.head_dim))).astype(np.float32)
        path = tmp_path / f"layer-{layer}.npz"
        np.savez(path, wq=wq, wk=wk)
        sha = hashlib.sha256(path.read_bytes()).hexdigest()
        entries.append(dict(layer_index=layer, initial_file=path.name, final_file=path.name, initial_sha256=sha,
                            final_sha256=sha))
    meta = dict(model_id="tiny-test", revision="fixture", r=r, layers=entries)
    meta["bank_id"] = hashlib.sha256(json.dumps(meta, sort_keys=True).encode()).hexdigest()
    return meta


def resign(meta):
    meta["bank_id"] = bank_id(meta)
    return meta


def test_load_bank_reads_the_files_and_folds_the_scale(tmp_path):
    meta = write_bank(tmp_path)
    bank = load_bank(tmp_path, meta, GEO, device="cpu")
    assert len(bank.indexes) == 2
    with np.load(tmp_path / "layer-1.npz", allow_pickle=False) as f:
        wq, wk = f["wq"], f["wk"]
    idx = bank.indexes[1]
    assert idx.wq.dtype == idx.wk.dtype == idx.wq_t_scaled.dtype == torch.float32
    assert np.array_equal(idx.wk.numpy(), wk)
    # wq_t_scaled[g, f, j] = wq[g, j, f] / sqrt(r), the reference's fold (indexer.py:45; trained.py:18)
    assert np.array_equal(idx.wq_t_scaled.numpy(), np.transpose(wq / np.float32(math.sqrt(R)), (0, 2, 1)))
    assert idx.identity == hashlib.sha256((tmp_path / "layer-1.npz").read_bytes()).hexdigest()
    again = load_bank(tmp_path, meta, GEO, device="cpu")
    assert again.identity == bank.identity
    initial = load_bank(tmp_path, meta, GEO, device="cpu", initial=True)
    assert initial.identity != bank.identity          # the role is part of the identity


@pytest.mark.parametrize("tamper,match", [
    (lambda m, p: m.update(revision="other"), "metadata identity mismatch"),
    (lambda m, p: resign(m) if m["layers"].pop() else None, "incomplete index bank"),
    (lambda m, p: resign(m) if m["layers"][0].update(final_file="../outside.npz") is None else None,
     "parameter path outside run"),
    (lambda m, p: (p / "layer-0.npz").write_bytes((p / "layer-0.npz").read_bytes() + b"changed"),
     "parameter file hash mismatch"),
])
def test_load_bank_rejects(tmp_path, tamper, match):
    meta = write_bank(tmp_path)
    tamper(meta, tmp_path)
    with pytest.raises(ValueError, match=match):
        load_bank(tmp_path, meta, GEO, device="cpu")


def test_load_bank_rejects_geometry_and_nonfinite(tmp_path):
    meta = write_bank(tmp_path)
    with pytest.raises(ValueError, match="geometry differs"):
        load_bank(tmp_path, meta, SimpleNamespace(layers=2, groups=2, heads_per_group=2, head_dim=8), device="cpu")
    path = tmp_path / "layer-0.npz"
    with np.load(path, allow_pickle=False) as f:
        wq, wk = f["wq"].copy(), f["wk"].copy()
    wk[0, 0, 0] = np.nan
    np.savez(path, wq=wq, wk=wk)
    sha = hashlib.sha256(path.read_bytes()).hexdigest()
    meta["layers"][0].update(final_sha256=sha)
    with pytest.raises(ValueError, match="nonfinite parameters"):
        load_bank(tmp_path, resign(meta), GEO, device="cpu")


def test_frozen_indexer_is_float32_only_and_notices_edits():
    wq = np.zeros((2, R, 32), np.float32)
    wk = np.zeros((2, R, 16), np.float32)
    with pytest.raises(ValueError, match="must be float32"):
        FrozenIndexer(wq.astype(np.float64), wk, identity="x", device="cpu")
    idx = FrozenIndexer(wq, wk, identity="x", device="cpu")
    idx.verify()
    idx.wk.add_(0.01)
    with pytest.raises(RuntimeError, match="parameters changed"):
        idx.verify()


def fake_state(indexers, *, has_index=True, index_dtype=torch.float32, valid_length=0, identity=None):
    cache = SimpleNamespace(has_index=has_index, index_dtype=index_dtype, device=torch.device("cpu"),
                            valid_length=valid_length)
    if identity is not None:
        cache.index_identity = identity
    return SimpleNamespace(indexers=indexers, cache=cache)


def test_guard(tmp_path):
    bank = load_bank(tmp_path, write_bank(tmp_path), GEO, device="cpu")
    st = fake_state(bank.indexes)
    bank.guard(st)
    assert st.cache.index_identity == bank.identity                       # an empty cache is bound to the bank
    bank.guard(fake_state(bank.indexes, valid_length=10, identity=bank.identity))
    with pytest.raises(RuntimeError, match="different parameter identity"):
        bank.guard(fake_state(bank.indexes, valid_length=10, identity="someone else"))
    with pytest.raises(RuntimeError, match="float32 index cache"):
        bank.guard(fake_state(bank.indexes, index_dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="float32 index cache"):
        bank.guard(fake_state(bank.indexes, has_index=False))
    other = FrozenBank(list(bank.indexes), identity="other")
    with pytest.raises(RuntimeError, match="state index bank changed"):
        other.guard(fake_state(list(reversed(bank.indexes))))
