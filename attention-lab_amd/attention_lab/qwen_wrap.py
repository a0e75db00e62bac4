"""Qwen3 on the HIP read path: a static K/V + index-table cache, per-layer attention wrappers and the prefill / decode
driver. The public surface is the reference's (src/attention_lab/qwen_wrap.py:52-615: LabCache, StepPlan,
build_step_plan, LabState, StateHolder, LabAttention, make_cache / make_indexers / make_state, wrap_model /
unwrap_model / is_wrapped, LabRunner, NativeRunner, tiny_qwen3, hf_cache_kv), with its phases and error types, so a
caller switches by import.

How this build arranges it:

* Storage. Each tensor kind is one allocation across layers ([layers, B, G, slots, d] for K and V, [layers, B, G, r,
  slots] for the index table); `cache.k[l]` etc. are views of it. `slots` is the capacity rounded up to a multiple
  of 8, so every index-table row starts 16 bytes aligned for the score kernels' 16-byte loads. An `_AppendLedger`
  enforces one append per layer per forward and commits the legal length once every layer has appended.
* Reads. A layer's forward computes its features once (q_pre / k_pre before RoPE for the index, q_main / k_main after
  the model's own RoPE for attention), then dispatches on the runner's explicit phase: prefill reads every legal
  position on the causal MFMA kernel and writes the chunk's index keys into the table in place
  (attnlab_project_keys); a dense decode step reads every legal position on the dense decode kernel; a sparse decode
  step asks the state's selector strategy for its read. The index selector (D0) is one fused HIP step per layer
  (z column, u, scan, top-k, gather-free attend); the recent (B) and uniform (C) selectors build their row list on
  the host, as the reference does, and read it with the gather-free attend.
* Plans. F and the candidate domain of a step are built once per step (`build_step_plan`) from device tensors the
  cache keeps, and tagged as the selection rule's F so the HIP step takes them without a device read.

Projections, q_norm / k_norm, RoPE, MLP, norms, embeddings and lm_head are the installed transformers model's. The
K/V cache must be bfloat16 with head_dim 128 for the kernels (other dtypes raise from the ops); the index table is
bfloat16, or float32 for a trained bank (trained.py). A token's slot is its absolute position; a rollback shortens the
legal range and leaves the old suffix in memory where no read or selection reaches it.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch
from torch import nn

from .decode import (gathered_decode_step_kernel, select_rows_recent, select_rows_uniform, sparse_decode_step_kernel,
                     tag_standard_f)
from .full import full_attention
from .indexer import GroupedIndexer, project_keys
from .selection import FIXED_PREFIX, FIXED_RECENT, fixed_budget, selection_layout
from .sparse import row_offsets

try:  # transformers is needed by this module only; the rest of the package imports without it
    from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb
except ImportError as _e:  # pragma: no cover
    apply_rotary_pos_emb = None
    _TRANSFORMERS_IMPORT_ERROR = _e

# Qwen3Model.forward builds no mask when attention_mask is already a mapping: the wrapper masks by legal length itself
MASK_BYPASS = {"full_attention": None}
SELECTORS = ("index", "recent", "uniform")   # D0, B, C
PHASES = ("prefill", "decode")
SLOT_ALIGN = 8   # rows per (b, g) are allocated in multiples of this: 16 bytes of a bfloat16 index-table row


# ---------------------------------------------------------------------------------------------------------------------
# cache
# ---------------------------------------------------------------------------------------------------------------------
@dataclass
class _AppendLedger:
    """Per-layer append counts and last writes, and the length of the forward in flight (None between forwards)."""
    layers: int
    writes: list = field(default_factory=list)
    last_write: list = field(default_factory=list)
    pending: int | None = None

    def __post_init__(self):
        self.writes = self.writes or [0] * self.layers
        self.last_write = self.last_write or [None] * self.layers

    def record(self, layer: int, start: int, length: int) -> None:
        if self.pending is None:
            self.pending = length
        elif self.pending != length:
            raise RuntimeError(f"layer {layer} appended {length} rows in a forward of {self.pending}")
        self.writes[layer] += 1
        self.last_write[layer] = (start, length)

    def commit(self, length: int) -> None:
        if self.pending != length:
            raise RuntimeError(f"advance({length}) does not match the appended length {self.pending}")
        if len(set(self.writes)) != 1:
            raise RuntimeError(f"unequal append counts across layers: {self.writes}")
        self.pending = None

    def copy(self) -> "_AppendLedger":
        return _AppendLedger(self.layers, list(self.writes), list(self.last_write), self.pending)


class LabCache:
    """Static per-layer K/V [B,G,slots,d] and optional index tables zT [B,G,r,slots] with one legal length for all
    layers (reference qwen_wrap.py:52-139). Allocated with torch.empty: slots at or past valid_length hold whatever the
    memory held (tests poison them) and no read or selection may touch them; slots past `capacity` are padding."""

    def __init__(self, *, layers: int, batch: int, groups: int, capacity: int, head_dim: int, index_dim=None, device,
                 dtype=torch.float32, index_dtype=None):
        if int(capacity) <= 0 or int(layers) <= 0:
            raise ValueError("capacity and layers must be positive")
        self.layers, self.batch, self.groups = int(layers), int(batch), int(groups)
        self.capacity, self.head_dim = int(capacity), int(head_dim)
        self.slots = -(-self.capacity // SLOT_ALIGN) * SLOT_ALIGN
        self.index_dim = None if index_dim is None else int(index_dim)
        self.device, self.dtype = torch.device(device), dtype
        self.index_dtype = dtype if index_dtype is None else index_dtype
        kv_shape = (self.layers, self.batch, self.groups, self.slots, self.head_dim)
        self._store = {"k": torch.empty(kv_shape, device=self.device, dtype=dtype),
                       "v": torch.empty(kv_shape, device=self.device, dtype=dtype)}
        if self.index_dim is not None:
            self._store["z"] = torch.empty(self.layers, self.batch, self.groups, self.index_dim, self.slots,
                                           device=self.device, dtype=self.index_dtype)
        self._bind_views()
        self.valid_length = 0
        self._ledger = _AppendLedger(self.layers)
        self.offsets = row_offsets(self.batch, self.groups, self.slots, self.device)   # [B,G,1] flat row offsets
        # the full fixed set's parts as flat row ids: the prefix, and the recent window relative to the legal length
        self.prefix_rows = (torch.arange(FIXED_PREFIX, device=self.device).view(1, 1, -1) + self.offsets).contiguous()
        self.recent_base = (torch.arange(-FIXED_RECENT, 0, device=self.device).view(1, 1, -1)
                            + self.offsets).contiguous()
        self.off_lo = (self.offsets + FIXED_PREFIX).contiguous()

    def _bind_views(self):
        self.k = list(self._store["k"].unbind(0))
        self.v = list(self._store["v"].unbind(0))
        self.z = list(self._store["z"].unbind(0)) if "z" in self._store else None

    @property
    def has_index(self) -> bool:
        return self.z is not None

    @property
    def writes(self) -> list:
        return self._ledger.writes

    @property
    def last_write(self) -> list:
        return self._ledger.last_write

    @property
    def _pending(self):
        return self._ledger.pending

    def reserve(self, layer: int, length: int) -> int:
        """Claim [valid_length, valid_length + length) for this layer's append and return its first slot."""
        start = self.valid_length
        if start + length > self.capacity:
            raise RuntimeError(f"cache capacity {self.capacity} exceeded: valid {start} + new {length}")
        self._ledger.record(layer, start, length)
        return start

    def append(self, layer: int, k_main: torch.Tensor, v: torch.Tensor, z=None) -> None:
        """Write this layer's T new rows at [valid_length, valid_length + T); exactly once per layer per forward."""
        T = int(k_main.shape[2])
        if z is not None and not self.has_index:
            raise RuntimeError("this cache was created without an index table")
        start = self.reserve(layer, T)
        self.k[layer][:, :, start:start + T].copy_(k_main)
        self.v[layer][:, :, start:start + T].copy_(v)
        if z is not None:
            self.z[layer][..., start:start + T].copy_(z)

    def advance(self, T: int) -> None:
        """Commit a forward of T tokens once every layer has appended it."""
        self._ledger.commit(int(T))
        self.valid_length += int(T)

    def rollback(self, length: int) -> None:
        """Shorten the legal range; the old suffix stays in memory, outside every read and selection."""
        if not 0 <= int(length) <= self.valid_length:
            raise ValueError(f"rollback to {length} outside [0, {self.valid_length}]")
        if self._ledger.pending is not None:
            raise RuntimeError("rollback during a forward")
        self.valid_length = int(length)

    def clone(self) -> "LabCache":
        """An independent branch: the same contents and ledger in storage of its own."""
        new = object.__new__(LabCache)
        new.__dict__.update(self.__dict__)
        new._store = {name: t.clone() for name, t in self._store.items()}
        new._bind_views()
        new._ledger = self._ledger.copy()
        return new

    def bytes(self) -> dict:
        """Bytes held (padding slots included)."""
        size = {name: t.numel() * t.element_size() for name, t in self._store.items()}
        kv, z = size["k"] + size["v"], size.get("z", 0)
        return {"kv_bytes": kv, "index_bytes": z, "total_bytes": kv + z}


# ---------------------------------------------------------------------------------------------------------------------
# step plan
# ---------------------------------------------------------------------------------------------------------------------
@dataclass
class StepPlan:
    """Selection shared by every layer of one decode step (reference qwen_wrap.py:143-165)."""
    legal_length: int          # [0, legal_length) is legal for this step's query, its own key included
    k0: int                    # the request's budget
    k: int                     # min(k0, candidates of this step)
    lo: int                    # candidate domain [lo, hi)
    hi: int
    fixed_count: int
    selected_count: int
    fixed_rows: torch.Tensor   # [B,G,F] flat row ids of F
    off_lo: torch.Tensor       # [B,G,1] row offsets + lo
    step_index: int = 0        # 0 for a request's first decode step
    shared_rows: torch.Tensor | None = None   # B: one row list for every layer of the step
    uniform_rng: object | None = None         # C: the step's numpy generator

    @property
    def write_col(self) -> int:
        return self.legal_length - 1

    @property
    def candidate_count(self) -> int:
        return self.hi - self.lo


def build_step_plan(cache: LabCache, legal_length: int, k0: int) -> StepPlan:
    """F and the candidate domain of a step whose legal range is [0, legal_length) (reference qwen_wrap.py:168-181)."""
    legal = int(legal_length)
    layout = selection_layout(legal)
    k = layout.clamp_k(k0)
    if legal >= FIXED_PREFIX + FIXED_RECENT:
        fixed_rows = torch.cat([cache.prefix_rows, cache.recent_base + legal], dim=-1)   # the full fixed set
        off_lo = cache.off_lo
    else:   # a short history: F is the whole legal range and nothing is a candidate
        fixed_rows = (torch.arange(legal, device=cache.device).view(1, 1, -1) + cache.offsets).contiguous()
        off_lo = (cache.offsets + layout.candidate_lo).contiguous()
    tag_standard_f(fixed_rows, off_lo, layout.candidate_lo, layout.candidate_hi, legal, cache.slots)
    return StepPlan(legal_length=legal, k0=int(k0), k=int(k), lo=layout.candidate_lo, hi=layout.candidate_hi,
                    fixed_count=layout.fixed_count, selected_count=layout.fixed_count + k, fixed_rows=fixed_rows,
                    off_lo=off_lo)


# ---------------------------------------------------------------------------------------------------------------------
# selectors of a sparse step: D0 (index), B (recent), C (uniform)
# ---------------------------------------------------------------------------------------------------------------------
class _IndexSelector:
    """D0: the fused HIP step scores the candidates, takes the top k, merges F and attends; it also writes the new
    key's index column."""
    writes_z = True

    def prepare(self, state, plan):
        pass

    def read(self, attn, state, plan, q5, q_pre, k_pre):
        l, cache = attn.layer_idx, state.cache
        idx = state.indexers[l]
        B, G, h, _, d = q5.shape
        res = sparse_decode_step_kernel(
            q5, q_pre.reshape(B, G, h, 1, d).to(idx.wk.dtype), cache.k[l], cache.v[l], cache.z[l], idx.wq_t_scaled,
            idx.wk, plan.fixed_rows, plan.off_lo, plan.lo, plan.hi, plan.k, plan.selected_count,
            k_pre_new=k_pre.to(idx.wk.dtype), write_col=plan.write_col, scale=attn.scaling,
            return_rows=state.record_selection, canonical_order=state.canonical_order)
        return res if state.record_selection else (res, None)


class _ListedSelector:
    """B and C: a host-built row list (F, then the chosen candidates), read by the gather-free attend."""
    writes_z = False

    def rows(self, state, plan):
        raise NotImplementedError

    def read(self, attn, state, plan, q5, q_pre, k_pre):
        l = attn.layer_idx
        rows = self.rows(state, plan)
        if state.canonical_order:
            B, G = q5.shape[:2]
            rows = rows.view(B, G, plan.selected_count).sort(dim=-1).values.reshape(-1)
        out = gathered_decode_step_kernel(q5, state.cache.k[l], state.cache.v[l], rows, plan.selected_count,
                                          scale=attn.scaling)
        return out, rows


class _RecentSelector(_ListedSelector):
    """B: the k most recent candidates, one list for every layer of the step (built once in prepare)."""

    def prepare(self, state, plan):
        plan.shared_rows = select_rows_recent(plan.fixed_rows, plan.off_lo, plan.lo, plan.hi, plan.k)

    def rows(self, state, plan):
        return plan.shared_rows


class _UniformSelector(_ListedSelector):
    """C: k candidates drawn without replacement per (b, g) from the step's seeded generator, per layer."""

    def prepare(self, state, plan):
        plan.uniform_rng = state.uniform_rng(plan.step_index)

    def rows(self, state, plan):
        return select_rows_uniform(plan.fixed_rows, plan.off_lo, plan.lo, plan.hi, plan.k, rng=plan.uniform_rng)


_SELECTOR_IMPL = {"index": _IndexSelector, "recent": _RecentSelector, "uniform": _UniformSelector}


# ---------------------------------------------------------------------------------------------------------------------
# state
# ---------------------------------------------------------------------------------------------------------------------
def _read_config_layers(cache: LabCache, indexers, mode: str, selector: str, sparse_layers):
    """Validate a read configuration against its cache and return the sparse layer set (None: every layer). The
    messages are the contract's; this function's own rule is that a configuration is checked in full before any state
    is built, cheapest property first."""
    problems = []
    if mode not in ("full", "sparse"):
        problems.append("mode must be 'full' or 'sparse'")
    if selector not in SELECTORS:
        problems.append(f"selector must be one of {SELECTORS}")
    if indexers is not None and len(indexers) != cache.layers:
        problems.append("one indexer per layer")
    if not problems and mode == "sparse" and selector == "index" and (indexers is None or not cache.has_index):
        problems.append("the index selector (D0) needs indexers and a cache with an index table")
    layers = None
    if sparse_layers is not None:
        layers = frozenset(int(x) for x in sparse_layers)
        if any(not 0 <= x < cache.layers for x in layers):
            problems.append("sparse layer index outside model")
    if problems:
        raise ValueError(problems[0])
    return layers


@dataclass
class _RequestBudget:
    """The budget of the request in flight. `number` counts the requests begun on a state, so the uniform selector's
    draws differ between requests; `start_length` is the legal length of the request's first decode step."""
    number: int = 0
    rho: float | None = None
    k0: int | None = None
    start_length: int | None = None

    def begin(self, valid_length: int, rho, k0) -> int:
        self.number += 1
        self.rho = None if rho is None else float(rho)
        self.start_length = int(valid_length) + 1
        self.k0 = fixed_budget(self.start_length, self.rho) if k0 is None else int(k0)
        return self.k0


class LabState:
    """One read configuration (reference qwen_wrap.py:189-256): the cache, the per-layer indexers, the mode (full or
    sparse), the selector of a sparse read and the plan and phase of the forward in flight. The request's budget
    (rho, k0, the first step's legal length, the request count) lives in a `_RequestBudget`; the reference's attribute
    names read through to it."""

    def __init__(self, cache: LabCache, indexers=None, *, mode: str = "full", selector: str = "index",
                 decode_backend: str = "sdpa_fold", prefill_backend: str = "sdpa_fold", uniform_seed: int = 0,
                 sparse_layers=None, cache_guard=None, canonical_order=False):
        self.sparse_layers = _read_config_layers(cache, indexers, mode, selector, sparse_layers)
        self.cache, self.indexers = cache, indexers
        self.mode, self.selector = mode, selector
        self.selector_impl = _SELECTOR_IMPL[selector]()
        self.decode_backend, self.prefill_backend = decode_backend, prefill_backend
        self.uniform_seed = int(uniform_seed)
        self.cache_guard = cache_guard
        self.canonical_order = bool(canonical_order)
        self.request = _RequestBudget()
        self.record_selection = False     # keep each layer's flat row list of the step in last_rows
        self.last_rows: list = [None] * cache.layers
        self.plan: StepPlan | None = None
        self.phase: str | None = None     # set by LabRunner before each forward, never inferred

    # the reference's names for the request budget
    rho = property(lambda self: self.request.rho)
    k0 = property(lambda self: self.request.k0)
    request_start_length = property(lambda self: self.request.start_length)
    request_counter = property(lambda self: self.request.number)

    def reads_sparse(self, layer: int) -> bool:
        return self.mode == "sparse" and (self.sparse_layers is None or layer in self.sparse_layers)

    def uniform_rng(self, step_index: int):
        """The uniform selector's generator for one step: PCG64 over the seed sequence (seed, request, step), so a
        step replayed after a rollback draws the same rows and no two (request, step) pairs share a stream (the
        reference's numpy default_rng([seed, request, step]), qwen_wrap.py:222-227)."""
        import numpy as np
        seq = np.random.SeedSequence([self.uniform_seed, self.request.number, int(step_index)])
        return np.random.Generator(np.random.PCG64(seq))

    def begin_request(self, rho: float, *, k0=None) -> int:
        """Fix k0 from the legal length of the request's first decode step (prefilled tokens + 1); an explicit k0
        overrides the rho rule (k0 = capacity selects every candidate, the sparse == full diagnostic)."""
        return self.request.begin(self.cache.valid_length, rho, k0)


class StateHolder:
    """The state the wrapped layers read, swappable between forwards."""

    def __init__(self, state: LabState | None = None):
        self.state = state


# ---------------------------------------------------------------------------------------------------------------------
# the wrapped attention
# ---------------------------------------------------------------------------------------------------------------------
class LabAttention(nn.Module):
    """A Qwen3Attention with its own projections, norms, RoPE and output path; only the read differs. `inner` is the
    original module (its parameters are used in place)."""

    def __init__(self, inner: nn.Module, holder: StateHolder, layer_idx: int):
        super().__init__()
        if apply_rotary_pos_emb is None:  # pragma: no cover
            raise _TRANSFORMERS_IMPORT_ERROR
        cfg = inner.config
        heads, groups = int(cfg.num_attention_heads), int(cfg.num_key_value_heads)
        if heads % groups:
            raise ValueError("query heads must be a multiple of KV heads")
        self.inner, self.holder, self.layer_idx = inner, holder, int(layer_idx)
        self.num_heads, self.num_groups, self.head_dim = heads, groups, int(inner.head_dim)
        self.heads_per_group = heads // groups
        self.scaling = float(inner.scaling)
        self.is_causal = True

    def _features(self, hidden_states, position_embeddings):
        """(q_pre, k_pre, v, q_main, k_main): q/k after q_norm / k_norm and before RoPE (the index features), then
        after the model's RoPE (what attention and the cache use). Shapes [B, H|G, T, d]."""
        inner = self.inner
        B, T, _ = hidden_states.shape
        shape = (B, T, -1, self.head_dim)
        q_pre = inner.q_norm(inner.q_proj(hidden_states).view(shape)).transpose(1, 2)
        k_pre = inner.k_norm(inner.k_proj(hidden_states).view(shape)).transpose(1, 2)
        v = inner.v_proj(hidden_states).view(shape).transpose(1, 2)
        cos, sin = position_embeddings
        q_main, k_main = apply_rotary_pos_emb(q_pre, k_pre, cos, sin)
        return q_pre, k_pre, v, q_main, k_main

    def _write_keys(self, st: LabState, k_main, v, k_pre) -> int:
        """Append this layer's K/V rows and, when the cache has an index table and the state its indexers, write the
        chunk's index keys z = Wk.k_pre straight into the table. Returns the first slot written."""
        l, cache = self.layer_idx, st.cache
        T = int(k_main.shape[2])
        start = cache.reserve(l, T)
        cache.k[l][:, :, start:start + T].copy_(k_main)
        cache.v[l][:, :, start:start + T].copy_(v)
        if cache.has_index and st.indexers is not None:
            wk = st.indexers[l].wk
            project_keys(k_pre.to(wk.dtype), wk, out=cache.z[l], col0=start)
        return start

    def _read_prefill(self, st, q5, k_pre, k_main, v):
        start = self._write_keys(st, k_main, v, k_pre)
        l, T = self.layer_idx, int(q5.shape[3])
        return full_attention(q5, st.cache.k[l], st.cache.v[l], valid_length=start + T, backend=st.prefill_backend,
                              scale=self.scaling)

    def _read_decode(self, st, q5, q_pre, k_pre, k_main, v):
        if q5.shape[3] != 1:
            raise RuntimeError("a decode step takes exactly one new token")
        l, cache = self.layer_idx, st.cache
        if not st.reads_sparse(l):
            start = self._write_keys(st, k_main, v, k_pre)
            return full_attention(q5, cache.k[l], cache.v[l], valid_length=start + 1, backend=st.decode_backend,
                                  scale=self.scaling)
        plan = st.plan
        if plan is None or plan.legal_length != cache.valid_length + 1:
            raise RuntimeError("sparse decode needs a StepPlan built for this step's legal length")
        impl = st.selector_impl
        if impl.writes_z:
            cache.append(l, k_main, v)   # K/V here; the fused step writes the new key's index column
        else:
            self._write_keys(st, k_main, v, k_pre)
        out, rows = impl.read(self, st, plan, q5, q_pre, k_pre)
        if st.record_selection:
            st.last_rows[l] = rows
        return out

    def forward(self, hidden_states, position_embeddings, attention_mask=None, past_key_values=None, **kwargs):
        st = self.holder.state
        if st is None:
            raise RuntimeError("no LabState set on the wrapped model")
        if st.phase not in PHASES:
            raise RuntimeError("LabState.phase must be 'prefill' or 'decode' (set by LabRunner.prefill / "
                               "LabRunner.step); the phase is never inferred from the input length")
        B, T, _ = hidden_states.shape
        q_pre, k_pre, v, q_main, k_main = self._features(hidden_states, position_embeddings)
        G, h, d = self.num_groups, self.heads_per_group, self.head_dim
        q5 = q_main.reshape(B, G, h, T, d)   # head g*h + i reads KV group g
        if st.phase == "prefill":
            out = self._read_prefill(st, q5, k_pre, k_main, v)
        else:
            out = self._read_decode(st, q5, q_pre, k_pre, k_main, v)
        attn = out.reshape(B, self.num_heads, T, d).transpose(1, 2).reshape(B, T, self.num_heads * d)
        return self.inner.o_proj(attn), None


# ---------------------------------------------------------------------------------------------------------------------
# model helpers
# ---------------------------------------------------------------------------------------------------------------------
@dataclass(frozen=True)
class ModelGeometry:
    layers: int
    hidden: int
    heads: int
    groups: int
    head_dim: int
    vocab: int
    max_positions: int

    @property
    def heads_per_group(self) -> int:
        return self.heads // self.groups


def _inner_attention(layer):
    attn = layer.self_attn
    return attn.inner if isinstance(attn, LabAttention) else attn


def geometry_of(model) -> ModelGeometry:
    """The attention geometry the config states (reference qwen_wrap.py:351-366), checked against layer 0's parameter
    shapes: a config edited after the weights were built is caught here, not inside a kernel."""
    cfg = model.config
    attn = _inner_attention(model.model.layers[0])
    geo = ModelGeometry(layers=len(model.model.layers), hidden=int(cfg.hidden_size),
                        heads=int(cfg.num_attention_heads), groups=int(cfg.num_key_value_heads),
                        head_dim=int(attn.head_dim), vocab=int(cfg.vocab_size),
                        max_positions=int(cfg.max_position_embeddings))
    q_width, kv_width = geo.heads * geo.head_dim, geo.groups * geo.head_dim
    implied = {"q_proj": (q_width, geo.hidden), "k_proj": (kv_width, geo.hidden), "v_proj": (kv_width, geo.hidden),
               "o_proj": (geo.hidden, q_width)}
    wrong = [(name, tuple(getattr(attn, name).weight.shape), want) for name, want in implied.items()
             if tuple(getattr(attn, name).weight.shape) != want]
    if wrong:
        name, got, want = wrong[0]
        raise ValueError(f"{name} weight shape {got} != {want} implied by the config")
    if {tuple(attn.q_norm.weight.shape), tuple(attn.k_norm.weight.shape)} != {(geo.head_dim,)}:
        raise ValueError("q_norm / k_norm act on head_dim in Qwen3; shapes disagree")
    return geo


def _param_device_dtype(model, device, dtype):
    p = next(model.parameters())
    return (p.device if device is None else device), (p.dtype if dtype is None else dtype)


def make_cache(model, capacity: int, *, with_index: bool, index_dim: int = 32, batch: int = 1, dtype=None, device=None,
               index_dtype=None) -> LabCache:
    geo = geometry_of(model)
    device, dtype = _param_device_dtype(model, device, dtype)
    return LabCache(layers=geo.layers, batch=batch, groups=geo.groups, capacity=capacity, head_dim=geo.head_dim,
                    index_dim=index_dim if with_index else None, device=device, dtype=dtype, index_dtype=index_dtype)


def make_indexers(model, *, r: int = 32, seed: int = 0, dtype=None, device=None) -> list[GroupedIndexer]:
    """One untrained grouped indexer per layer, layer l seeded seed * 1000 + l (the reference's seeds)."""
    geo = geometry_of(model)
    device, dtype = _param_device_dtype(model, device, dtype)
    return [GroupedIndexer(geo.groups, geo.heads_per_group, geo.head_dim, r, device=device, dtype=dtype,
                           seed=seed * 1000 + layer) for layer in range(geo.layers)]


def make_state(model, capacity: int, mode: str, *, selector: str = "index", r: int = 32, seed: int = 0, batch: int = 1,
               **kw) -> LabState:
    """A: mode "full". D0: mode "sparse" with the index selector (index table and indexers). B / C: mode "sparse" with
    selector "recent" / "uniform" (neither an index table nor indexers)."""
    indexed = mode == "sparse" and selector == "index"
    cache = make_cache(model, capacity, with_index=indexed, index_dim=r, batch=batch)
    return LabState(cache, make_indexers(model, r=r, seed=seed) if indexed else None, mode=mode, selector=selector,
                    **kw)


def is_wrapped(model) -> bool:
    return isinstance(model.model.layers[0].self_attn, LabAttention)


def wrap_model(model, holder: StateHolder | None = None) -> StateHolder:
    """Put a LabAttention around every layer's self_attn (the original module is kept inside); returns the holder."""
    if is_wrapped(model):
        raise RuntimeError("model is already wrapped")
    holder = StateHolder() if holder is None else holder
    for i, layer in enumerate(model.model.layers):
        layer.self_attn = LabAttention(layer.self_attn, holder, i)
    return holder


def unwrap_model(model) -> None:
    for layer in model.model.layers:
        layer.self_attn = _inner_attention(layer)


# ---------------------------------------------------------------------------------------------------------------------
# drivers
# ---------------------------------------------------------------------------------------------------------------------
def _chunks(T: int, chunk: int):
    if chunk <= 0:
        raise ValueError("chunk must be positive")
    return [(a, min(a + chunk, T)) for a in range(0, T, chunk)]


class LabRunner:
    """Prefill / decode driver of a wrapped model over one LabState (reference qwen_wrap.py:417-486). Every forward is
    the model's own (embeddings, layers, norm, lm_head); positions are slices of one preallocated arange."""

    def __init__(self, model, holder: StateHolder, state: LabState):
        if not is_wrapped(model):
            raise RuntimeError("wrap_model first")
        self.model, self.holder, self.state = model, holder, state
        self.positions = torch.arange(state.cache.capacity, device=state.cache.device)

    @property
    def cache(self) -> LabCache:
        return self.state.cache

    def _plan_decode(self, st: LabState, legal: int) -> StepPlan | None:
        if st.mode != "sparse":
            return None
        if st.k0 is None:
            raise RuntimeError("call state.begin_request(rho) before the first sparse decode step")
        plan = build_step_plan(st.cache, legal, st.k0)
        plan.step_index = legal - st.request_start_length
        st.selector_impl.prepare(st, plan)
        return plan

    def forward(self, input_ids: torch.Tensor, *, phase: str, logits_to_keep: int = 1) -> torch.Tensor:
        """One model forward in an explicit phase: "prefill" (any chunk length: every legal position read, index keys
        written, nothing selected) or "decode" (one token, read by the state's mode)."""
        if phase not in PHASES:
            raise ValueError("phase must be 'prefill' or 'decode'")
        st = self.state
        cache = st.cache
        if st.cache_guard is not None:
            st.cache_guard(st)
        B, T = input_ids.shape
        if B != cache.batch:
            raise ValueError("batch size differs from the cache")
        if phase == "decode" and T != 1:
            raise ValueError("a decode step takes exactly one token per sequence")
        start = cache.valid_length
        st.plan = self._plan_decode(st, start + 1) if phase == "decode" else None
        st.phase = phase
        self.holder.state = st
        out = self.model(input_ids=input_ids, position_ids=self.positions[start:start + T].unsqueeze(0),
                         attention_mask=MASK_BYPASS, use_cache=False, logits_to_keep=logits_to_keep)
        cache.advance(T)
        return out.logits

    def prefill(self, input_ids: torch.Tensor, chunk: int, *, keep_logits: bool = False):
        """The prompt in chunks of `chunk` tokens, every chunk a prefill forward."""
        logits = [self.forward(input_ids[:, a:b], phase="prefill", logits_to_keep=0 if keep_logits else 1)
                  for a, b in _chunks(input_ids.shape[1], chunk)]
        return torch.cat(logits, dim=1) if keep_logits else logits[-1]

    def step(self, token_ids: torch.Tensor) -> torch.Tensor:
        """One decode step: [B, 1] token ids -> [B, 1, V] next-token logits."""
        if token_ids.shape[1] != 1:
            raise ValueError("a decode step takes one token per sequence")
        return self.forward(token_ids, phase="decode", logits_to_keep=1)

    def rollback(self, length: int) -> None:
        self.state.cache.rollback(length)


class NativeRunner:
    """The unwrapped model on transformers' own cache and attention: the comparison target of the wrapper's full read
    (reference qwen_wrap.py:489-531). None of this build's kernels run here."""

    def __init__(self, model, cache, capacity: int):
        if is_wrapped(model):
            raise RuntimeError("NativeRunner needs the unwrapped model")
        self.model, self.cache = model, cache
        self.length = 0
        self.positions = torch.arange(int(capacity), device=next(model.parameters()).device)

    def forward(self, input_ids: torch.Tensor, *, logits_to_keep: int = 1) -> torch.Tensor:
        T = input_ids.shape[1]
        out = self.model(input_ids=input_ids, position_ids=self.positions[self.length:self.length + T].unsqueeze(0),
                         past_key_values=self.cache, use_cache=True, logits_to_keep=logits_to_keep)
        self.length += T
        return out.logits

    def prefill(self, input_ids: torch.Tensor, chunk: int, *, keep_logits: bool = False):
        logits = [self.forward(input_ids[:, a:b], logits_to_keep=0 if keep_logits else 1)
                  for a, b in _chunks(input_ids.shape[1], chunk)]
        return torch.cat(logits, dim=1) if keep_logits else logits[-1]

    def step(self, token_ids: torch.Tensor) -> torch.Tensor:
        return self.forward(token_ids, logits_to_keep=1)

    def rollback(self, length: int) -> None:
        """Make the cache hold the first `length` tokens again. Each layer is shortened by its own kind: a layer
        preallocated to the capacity (transformers' static layer) keeps its storage and gets `length` as its written
        count, so attention masks the slots past it; a growing layer (the dynamic one) is cut back to its first
        `length` positions."""
        length = int(length)
        if length > self.length:
            raise ValueError("cannot roll forward")
        if length < self.length:
            for lay in self.cache.layers:
                _shorten_layer(lay, length)
        self.length = length


def _shorten_layer(lay, length: int) -> None:
    written = getattr(lay, "cumulative_length", None)
    if isinstance(written, torch.Tensor):
        written.fill_(length)
    elif isinstance(getattr(lay, "keys", None), torch.Tensor):
        lay.keys = lay.keys[..., :length, :]
        lay.values = lay.values[..., :length, :]
    else:
        raise TypeError(f"cannot roll back a cache layer of type {type(lay).__name__}")


def tiny_qwen3(*, seed: int = 0, layers: int = 2, hidden: int = 64, heads: int = 4, groups: int = 2, head_dim: int = 16,
               intermediate: int = 128, vocab: int = 256, max_positions: int = 2048, dtype=torch.float64):
    """A randomly initialised Qwen3 from a local config (nothing is downloaded). The HIP kernels need head_dim 128 and
    bfloat16; the defaults are the reference's CPU test model."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=vocab, hidden_size=hidden, intermediate_size=intermediate, num_hidden_layers=layers,
                      num_attention_heads=heads, num_key_value_heads=groups, head_dim=head_dim,
                      max_position_embeddings=max_positions, tie_word_embeddings=False, attn_implementation="sdpa")
    torch.manual_seed(seed)
    model = Qwen3ForCausalLM(cfg).to(dtype).eval()
    for p in model.parameters():
        p.requires_grad_(False)
    return model


def hf_cache_kv(cache, layer: int):
    """K/V [B,G,L,d] a transformers cache holds for one layer (the static cache's comparison target)."""
    lay = cache.layers[layer]
    return lay.keys, lay.values
