"""Qwen3 integration on the HIP path: every layer's self_attn wrapped around the frozen body, a static K/V cache with an
index table, and prefill / decode drivers (counterpart of src/attention_lab/qwen_wrap.py:52-486).

The names, arguments, phases and errors are the reference's, so a caller of `LabCache` / `LabState` / `LabRunner`
switches by import. The projections, q_norm / k_norm, the model's own RoPE (transformers' apply_rotary_pos_emb),
embeddings, MLP, norms and lm_head are the installed model's, untouched. What runs on this build's kernels:

- sparse decode, index selector (D0): `decode.sparse_decode_step_kernel`, i.e. one `attnlab_sparse_decode_step` per
  layer (z column of the new key, u, scan, top-k, gather-free attend);
- sparse decode, recent (B) / uniform (C) selectors: the row list is built on the host as in the reference and read
  by the gather-free attend (`decode.gathered_decode_step_kernel`);
- dense decode (A): the dense decode kernel (`full.full_attention`, one query);
- prefill: `full.full_attention` over the chunk's queries (one dense-decode launch per query position, causal) and
  the index table filled by `attnlab_project_keys`.

The K/V cache must be bfloat16 with head_dim 128 and r <= 32 (what the kernels take); the index table is bfloat16,
or float32 for a trained bank (trained.py:78-81). Anything else raises from the op.

Per layer, as in the reference (its docs/IMPLEMENTATION.md §1): hidden -> q/k/v_proj -> q_norm / k_norm -> (q_pre,
k_pre, index features before RoPE) -> RoPE -> (q_main, k_main) -> append k_main, v (and z = Wk.k_pre) exactly once ->
read -> o_proj. A token's cache slot is its absolute position; rows are read by original position; a rollback leaves
the old suffix in memory outside the legal range, where it can be neither read nor selected.
"""
from __future__ import annotations

from dataclasses import dataclass

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

# Qwen3Model.forward builds no mask when attention_mask is already a mapping (the wrapper masks by legal length)
MASK_BYPASS = {"full_attention": None}

SELECTORS = ("index", "recent", "uniform")   # D0 / B / C
SLOT_ALIGN = 8   # cache rows per (b, g) are allocated in multiples of this (16 bytes of a bf16 index-table row)


class LabCache:
    """Per-layer K/V [B,G,C,d] and optional index tables zT [B,G,r,C], one legal length shared by all layers. In memory
    C is `slots`, the capacity rounded up to a multiple of SLOT_ALIGN; positions at or past `capacity` are never used.

    Allocated with torch.empty: slots at or beyond valid_length hold garbage (tests poison them with NaN) and no read
    or selection may touch them.
    """

    def __init__(self, *, layers: int, batch: int, groups: int, capacity: int, head_dim: int, index_dim=None, device,
                 dtype=torch.float32, index_dtype=None):
        if int(capacity) <= 0 or int(layers) <= 0:
            raise ValueError("capacity and layers must be positive")
        self.layers, self.batch, self.groups = int(layers), int(batch), int(groups)
        self.capacity, self.head_dim = int(capacity), int(head_dim)
        # rows per (b, g) in memory: the capacity rounded up to a multiple of SLOT_ALIGN, so every index-table row
        # starts 16 bytes aligned and the score kernels take their 16-byte loads whatever the capacity; the slots
        # past `capacity` are never written or read
        self.slots = -(-self.capacity // SLOT_ALIGN) * SLOT_ALIGN
        self.index_dim = None if index_dim is None else int(index_dim)
        self.device, self.dtype = torch.device(device), dtype
        self.index_dtype = dtype if index_dtype is None else index_dtype
        shape = (self.batch, self.groups, self.slots, self.head_dim)
        self.k = [torch.empty(shape, device=self.device, dtype=dtype) for _ in range(self.layers)]
        self.v = [torch.empty(shape, device=self.device, dtype=dtype) for _ in range(self.layers)]
        self.z = None if self.index_dim is None else [
            torch.empty(self.batch, self.groups, self.index_dim, self.slots, device=self.device, dtype=self.index_dtype)
            for _ in range(self.layers)]
        self.valid_length = 0
        self.offsets = row_offsets(self.batch, self.groups, self.slots, self.device)         # [B,G,1]
        self.prefix_rows = (torch.arange(FIXED_PREFIX, device=self.device).view(1, 1, -1) + self.offsets).contiguous()
        self.recent_base = (torch.arange(-FIXED_RECENT, 0, device=self.device).view(1, 1, -1)
                            + self.offsets).contiguous()
        self.off_lo = (self.offsets + FIXED_PREFIX).contiguous()
        self.writes = [0] * self.layers          # appends per layer; exactly one per layer per forward
        self.last_write = [None] * self.layers   # (start, length) of each layer's latest append
        self._pending = None                     # length of the forward in flight

    @property
    def has_index(self) -> bool:
        return self.z is not None

    def append(self, layer: int, k_main: torch.Tensor, v: torch.Tensor, z=None) -> None:
        """Write this layer's T new rows at [valid_length, valid_length + T); once per layer per forward."""
        start, T = self.valid_length, int(k_main.shape[2])
        if start + T > self.capacity:
            raise RuntimeError(f"cache capacity {self.capacity} exceeded: valid {start} + new {T}")
        if self._pending is None:
            self._pending = T
        elif self._pending != T:
            raise RuntimeError("layers appended different lengths within one forward")
        self.k[layer][:, :, start:start + T].copy_(k_main)
        self.v[layer][:, :, start:start + T].copy_(v)
        if z is not None:
            if self.z is None:
                raise RuntimeError("this cache was created without an index table")
            self.z[layer][..., start:start + T].copy_(z)
        self.writes[layer] += 1
        self.last_write[layer] = (start, T)

    def advance(self, T: int) -> None:
        """Commit a forward of T tokens once every layer has appended exactly once."""
        if self._pending != int(T):
            raise RuntimeError(f"advance({T}) does not match the appended length {self._pending}")
        if any(w != self.writes[0] for w in self.writes):
            raise RuntimeError(f"unequal append counts across layers: {self.writes}")
        self.valid_length += int(T)
        self._pending = None

    def rollback(self, length: int) -> None:
        """Shrink the legal range; the old suffix stays in memory but is outside every read and selection."""
        if not 0 <= int(length) <= self.valid_length:
            raise ValueError(f"rollback to {length} outside [0, {self.valid_length}]")
        if self._pending is not None:
            raise RuntimeError("rollback during a forward")
        self.valid_length = int(length)

    def clone(self) -> "LabCache":
        """An independent copy (a request branch) sharing no storage with this one."""
        new = LabCache.__new__(LabCache)
        new.__dict__.update({key: val for key, val in self.__dict__.items()
                             if key not in ("k", "v", "z", "writes", "last_write")})
        new.k = [t.clone() for t in self.k]
        new.v = [t.clone() for t in self.v]
        new.z = None if self.z is None else [t.clone() for t in self.z]
        new.writes, new.last_write = list(self.writes), list(self.last_write)
        return new

    def bytes(self) -> dict:
        """Bytes the cache holds (its tensors, padding slots included)."""
        kv = sum(t.numel() * t.element_size() for t in self.k + self.v)
        z = 0 if self.z is None else sum(t.numel() * t.element_size() for t in self.z)
        return {"kv_bytes": kv, "index_bytes": z, "total_bytes": kv + z}


@dataclass
class StepPlan:
    """Selection plan shared by every layer of one decode step (reference qwen_wrap.py:143-165)."""
    legal_length: int          # positions [0, legal_length) are legal for this step's query, its own key included
    k0: int                    # fixed per request
    k: int                     # min(k0, candidates this step)
    lo: int                    # candidate domain [lo, hi)
    hi: int
    fixed_count: int
    selected_count: int
    fixed_rows: torch.Tensor   # [B,G,F] flat row ids of F
    off_lo: torch.Tensor       # [B,G,1] offsets + lo
    step_index: int = 0        # 0 for the request's first decode step
    shared_rows: torch.Tensor | None = None   # B: one row list for every layer, built once per step
    uniform_rng: object | None = None         # C: numpy Generator of this step

    @property
    def write_col(self) -> int:
        return self.legal_length - 1

    @property
    def candidate_count(self) -> int:
        return self.hi - self.lo


def build_step_plan(cache: LabCache, legal_length: int, k0: int) -> StepPlan:
    """F and the candidate domain for a step whose legal range is [0, legal_length) (reference qwen_wrap.py:168-181).
    With the full fixed set (legal >= 68) F is assembled from device tensors the cache keeps, without a host copy."""
    layout = selection_layout(legal_length)
    k = layout.clamp_k(k0)
    if layout.fixed_prefix == FIXED_PREFIX and layout.recent_start == legal_length - FIXED_RECENT:
        fixed_rows = torch.cat([cache.prefix_rows, cache.recent_base + legal_length], dim=-1)
        off_lo = cache.off_lo
    else:   # short history: F is (almost) everything
        pos = torch.tensor(layout.fixed_positions(), dtype=torch.long, device=cache.device).view(1, 1, -1)
        fixed_rows = (pos + cache.offsets).contiguous()
        off_lo = (cache.offsets + layout.candidate_lo).contiguous()
    tag_standard_f(fixed_rows, off_lo, layout.candidate_lo, layout.candidate_hi, int(legal_length), cache.slots)
    return StepPlan(legal_length=int(legal_length), k0=int(k0), k=int(k), lo=layout.candidate_lo,
                    hi=layout.candidate_hi, fixed_count=layout.fixed_count, selected_count=layout.fixed_count + k,
                    fixed_rows=fixed_rows, off_lo=off_lo)


class LabState:
    """One read configuration (reference qwen_wrap.py:189-256): cache, indexers, mode (full | sparse), the selector of
    a sparse read (index = D0, recent = B, uniform = C) and the plan of the step in flight."""

    def __init__(self, cache: LabCache, indexers=None, *, mode: str = "full", selector: str = "index",
                 decode_backend: str = "sdpa_fold", prefill_backend: str = "sdpa_fold", uniform_seed: int = 0,
                 sparse_layers=None, cache_guard=None, canonical_order=False):
        if mode not in ("full", "sparse"):
            raise ValueError("mode must be 'full' or 'sparse'")
        if selector not in SELECTORS:
            raise ValueError(f"selector must be one of {SELECTORS}")
        if mode == "sparse" and selector == "index" and (indexers is None or not cache.has_index):
            raise ValueError("the index selector (D0) needs indexers and a cache with an index table")
        if indexers is not None and len(indexers) != cache.layers:
            raise ValueError("one indexer per layer")
        self.cache, self.indexers, self.mode, self.selector = cache, indexers, mode, selector
        self.sparse_layers = None if sparse_layers is None else frozenset(sparse_layers)
        if self.sparse_layers is not None and not self.sparse_layers.issubset(range(cache.layers)):
            raise ValueError("sparse layer index outside model")
        self.cache_guard = cache_guard
        self.canonical_order = bool(canonical_order)
        self.decode_backend, self.prefill_backend = decode_backend, prefill_backend
        self.uniform_seed = int(uniform_seed)
        self.request_counter = 0           # begin_request bumps it, so C's draws differ between requests
        self.record_selection = False      # keep each layer's flat row list of the current step in last_rows
        self.last_rows: list = [None] * cache.layers
        self.plan: StepPlan | None = None
        self.phase: str | None = None      # "prefill" | "decode", set by LabRunner before each forward
        self.rho = None
        self.k0 = None
        self.request_start_length = None

    def uniform_rng(self, step_index: int):
        """C's generator of one decode step, seeded by (uniform_seed, request, step): a step replayed after a rollback
        draws the same rows, and no two (request, step) pairs share a stream."""
        import numpy as np
        return np.random.default_rng([self.uniform_seed, self.request_counter, int(step_index)])

    def begin_request(self, rho: float, *, k0=None) -> int:
        """Fix k0 from the legal length of the first decode step (prefilled tokens + the first new one). `k0` overrides
        the rho rule (diagnostics: k0 = capacity selects every candidate, so sparse must equal full)."""
        self.rho = None if rho is None else float(rho)
        self.request_start_length = self.cache.valid_length + 1
        self.k0 = fixed_budget(self.request_start_length, self.rho) if k0 is None else int(k0)
        self.request_counter += 1
        return self.k0


class StateHolder:
    """Mutable pointer, so one wrapped model can alternate between read configurations."""

    def __init__(self, state: LabState | None = None):
        self.state = state


class LabAttention(nn.Module):
    """Replacement for one Qwen3Attention with the same projections, norms, RoPE and output path; only the read
    differs. `inner` is the original module (its parameters are reused, never copied)."""

    def __init__(self, inner: nn.Module, holder: StateHolder, layer_idx: int):
        super().__init__()
        if apply_rotary_pos_emb is None:  # pragma: no cover
            raise _TRANSFORMERS_IMPORT_ERROR
        self.inner = inner
        self.holder = holder
        self.layer_idx = int(layer_idx)
        cfg = inner.config
        self.num_heads = int(cfg.num_attention_heads)
        self.num_groups = int(cfg.num_key_value_heads)
        self.head_dim = int(inner.head_dim)
        if self.num_heads % self.num_groups:
            raise ValueError("query heads must be a multiple of KV heads")
        self.heads_per_group = self.num_heads // self.num_groups
        self.scaling = float(inner.scaling)
        self.is_causal = True

    def _index_keys(self, st: LabState, k_pre):
        """z = Wk.k_pre of the new keys when the cache has an index table (prefill and dense decode fill it)."""
        if not (st.cache.has_index and st.indexers is not None):
            return None
        idx = st.indexers[self.layer_idx]
        return project_keys(k_pre.to(idx.wk.dtype), idx.wk)

    def forward(self, hidden_states, position_embeddings, attention_mask=None, past_key_values=None, **kwargs):
        inner, st = self.inner, self.holder.state
        if st is None:
            raise RuntimeError("no LabState set on the wrapped model")
        B, T, _ = hidden_states.shape
        shape = (B, T, -1, self.head_dim)
        q_pre = inner.q_norm(inner.q_proj(hidden_states).view(shape)).transpose(1, 2)   # [B,H,T,d], before RoPE
        k_pre = inner.k_norm(inner.k_proj(hidden_states).view(shape)).transpose(1, 2)   # [B,G,T,d], before RoPE
        v = inner.v_proj(hidden_states).view(shape).transpose(1, 2)                     # [B,G,T,d]
        cos, sin = position_embeddings
        q_main, k_main = apply_rotary_pos_emb(q_pre, k_pre, cos, sin)
        cache, l = st.cache, self.layer_idx
        L0 = cache.valid_length
        G, h, d = self.num_groups, self.heads_per_group, self.head_dim
        q5 = q_main.reshape(B, G, h, T, d)                                              # head g*h+i reads group g
        if st.phase not in ("prefill", "decode"):
            raise RuntimeError("LabState.phase must be 'prefill' or 'decode' (set by LabRunner.prefill / "
                               "LabRunner.step); the phase is never inferred from the input length")
        if st.phase == "decode":
            if T != 1:
                raise RuntimeError("a decode step takes exactly one new token")
            if st.mode == "sparse" and (st.sparse_layers is None or l in st.sparse_layers):
                plan = st.plan
                if plan is None or plan.legal_length != L0 + 1:
                    raise RuntimeError("sparse decode needs a StepPlan built for this step's legal length")
                cache.append(l, k_main, v)   # K/V once; D0 writes the new key's z column inside its step
                if st.selector == "index":
                    idx = st.indexers[l]
                    res = sparse_decode_step_kernel(
                        q5, q_pre.reshape(B, G, h, 1, d).to(idx.wk.dtype), cache.k[l], cache.v[l], cache.z[l],
                        idx.wq_t_scaled, idx.wk, plan.fixed_rows, plan.off_lo, plan.lo, plan.hi, plan.k,
                        plan.selected_count, k_pre_new=k_pre.to(idx.wk.dtype), write_col=plan.write_col,
                        scale=self.scaling, return_rows=st.record_selection, canonical_order=st.canonical_order)
                    out, rows = res if st.record_selection else (res, None)
                else:
                    if st.selector == "recent":
                        rows = plan.shared_rows
                    else:
                        rows = select_rows_uniform(plan.fixed_rows, plan.off_lo, plan.lo, plan.hi, plan.k,
                                                   rng=plan.uniform_rng)
                    if st.canonical_order:
                        rows = rows.view(B, G, plan.selected_count).sort(dim=-1).values.reshape(-1)
                    out = gathered_decode_step_kernel(q5, cache.k[l], cache.v[l], rows, plan.selected_count,
                                                      scale=self.scaling)
                if st.record_selection:
                    st.last_rows[l] = rows
            else:
                cache.append(l, k_main, v, self._index_keys(st, k_pre))
                out = full_attention(q5, cache.k[l], cache.v[l], valid_length=L0 + 1, backend=st.decode_backend,
                                     scale=self.scaling)
        else:   # prefill: the full read over every legal position, the index table filled; nothing is selected
            cache.append(l, k_main, v, self._index_keys(st, k_pre))
            out = full_attention(q5, cache.k[l], cache.v[l], valid_length=L0 + T, backend=st.prefill_backend,
                                 scale=self.scaling)
        attn = out.reshape(B, self.num_heads, T, d).transpose(1, 2).reshape(B, T, self.num_heads * d)
        return inner.o_proj(attn), None


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


def _attention_module(layer):
    return layer.self_attn.inner if isinstance(layer.self_attn, LabAttention) else layer.self_attn


def geometry_of(model) -> ModelGeometry:
    """The geometry from the config, checked against the actual parameter shapes."""
    cfg = model.config
    attn = _attention_module(model.model.layers[0])
    heads, groups, hidden = int(cfg.num_attention_heads), int(cfg.num_key_value_heads), int(cfg.hidden_size)
    head_dim = int(attn.head_dim)
    expect = {"q_proj": (heads * head_dim, hidden), "k_proj": (groups * head_dim, hidden),
              "v_proj": (groups * head_dim, hidden), "o_proj": (hidden, heads * head_dim)}
    for name, want in expect.items():
        got = tuple(getattr(attn, name).weight.shape)
        if got != want:
            raise ValueError(f"{name} weight shape {got} != {want} implied by the config")
    if tuple(attn.q_norm.weight.shape) != (head_dim,) or tuple(attn.k_norm.weight.shape) != (head_dim,):
        raise ValueError("q_norm / k_norm act on head_dim in Qwen3; shapes disagree")
    return ModelGeometry(layers=len(model.model.layers), hidden=hidden, heads=heads, groups=groups, head_dim=head_dim,
                         vocab=int(cfg.vocab_size), max_positions=int(cfg.max_position_embeddings))


def make_cache(model, capacity: int, *, with_index: bool, index_dim: int = 32, batch: int = 1, dtype=None, device=None,
               index_dtype=None) -> LabCache:
    geo = geometry_of(model)
    p = next(model.parameters())
    return LabCache(layers=geo.layers, batch=batch, groups=geo.groups, capacity=capacity, head_dim=geo.head_dim,
                    index_dim=index_dim if with_index else None, device=p.device if device is None else device,
                    dtype=p.dtype if dtype is None else dtype, index_dtype=index_dtype)


def make_indexers(model, *, r: int = 32, seed: int = 0, dtype=None, device=None) -> list[GroupedIndexer]:
    """One untrained grouped indexer per layer, seeded seed * 1000 + layer as in the reference."""
    geo = geometry_of(model)
    p = next(model.parameters())
    return [GroupedIndexer(geo.groups, geo.heads_per_group, geo.head_dim, r,
                           device=p.device if device is None else device, dtype=p.dtype if dtype is None else dtype,
                           seed=seed * 1000 + i) for i in range(geo.layers)]


def make_state(model, capacity: int, mode: str, *, selector: str = "index", r: int = 32, seed: int = 0, batch: int = 1,
               **kw) -> LabState:
    """A: mode "full". D0: mode "sparse", selector "index" (index table + indexers). B / C: mode "sparse" with
    selector "recent" / "uniform" (no index table, no indexers)."""
    with_index = mode == "sparse" and selector == "index"
    cache = make_cache(model, capacity, with_index=with_index, index_dim=r, batch=batch)
    idx = make_indexers(model, r=r, seed=seed) if with_index else None
    return LabState(cache, idx, mode=mode, selector=selector, **kw)


def wrap_model(model, holder: StateHolder | None = None) -> StateHolder:
    """Replace every layer's self_attn with LabAttention around the original module; returns the shared holder."""
    holder = StateHolder() if holder is None else holder
    for i, layer in enumerate(model.model.layers):
        if isinstance(layer.self_attn, LabAttention):
            raise RuntimeError("model is already wrapped")
        layer.self_attn = LabAttention(layer.self_attn, holder, i)
    return holder


def unwrap_model(model) -> None:
    for layer in model.model.layers:
        if isinstance(layer.self_attn, LabAttention):
            layer.self_attn = layer.self_attn.inner


def is_wrapped(model) -> bool:
    return isinstance(model.model.layers[0].self_attn, LabAttention)


class LabRunner:
    """Prefill / decode driver of a wrapped model and one LabState (reference qwen_wrap.py:417-486). Every forward is
    the model's own (embeddings -> layers -> norm -> lm_head); positions are views of one preallocated arange."""

    def __init__(self, model, holder: StateHolder, state: LabState):
        if not is_wrapped(model):
            raise RuntimeError("wrap_model first")
        self.model, self.holder, self.state = model, holder, state
        self.positions = torch.arange(state.cache.capacity, device=state.cache.device)

    @property
    def cache(self) -> LabCache:
        return self.state.cache

    def forward(self, input_ids: torch.Tensor, *, phase: str, logits_to_keep: int = 1) -> torch.Tensor:
        """One model forward. "prefill": every legal position is read and the index table filled (any chunk size);
        "decode": one new token read by the state's mode."""
        if phase not in ("prefill", "decode"):
            raise ValueError("phase must be 'prefill' or 'decode'")
        st, cache = self.state, self.state.cache
        if st.cache_guard is not None:
            st.cache_guard(st)
        B, T = input_ids.shape
        if B != cache.batch:
            raise ValueError("batch size differs from the cache")
        start = cache.valid_length
        st.phase = phase
        st.plan = None
        if phase == "decode":
            if T != 1:
                raise ValueError("a decode step takes exactly one token per sequence")
            if st.mode == "sparse":
                if st.k0 is None:
                    raise RuntimeError("call state.begin_request(rho) before the first sparse decode step")
                plan = build_step_plan(cache, start + 1, st.k0)
                plan.step_index = start + 1 - st.request_start_length
                if st.selector == "recent":
                    plan.shared_rows = select_rows_recent(plan.fixed_rows, plan.off_lo, plan.lo, plan.hi, plan.k)
                elif st.selector == "uniform":
                    plan.uniform_rng = st.uniform_rng(plan.step_index)
                st.plan = plan
        self.holder.state = st
        out = self.model(input_ids=input_ids, position_ids=self.positions[start:start + T].unsqueeze(0),
                         attention_mask=MASK_BYPASS, use_cache=False, logits_to_keep=logits_to_keep)
        cache.advance(T)
        return out.logits

    def prefill(self, input_ids: torch.Tensor, chunk: int, *, keep_logits: bool = False):
        """Dense prefill in chunks (the index table is filled chunk by chunk when the cache has one)."""
        if chunk <= 0:
            raise ValueError("chunk must be positive")
        T = input_ids.shape[1]
        outs, logits = [], None
        for a in range(0, T, chunk):
            logits = self.forward(input_ids[:, a:a + chunk], phase="prefill", logits_to_keep=0 if keep_logits else 1)
            if keep_logits:
                outs.append(logits)
        return torch.cat(outs, dim=1) if keep_logits else logits

    def step(self, token_ids: torch.Tensor) -> torch.Tensor:
        """One decode step: token ids [B,1] -> scores [B,1,V] of the next token."""
        if token_ids.shape[1] != 1:
            raise ValueError("a decode step takes one token per sequence")
        return self.forward(token_ids, phase="decode", logits_to_keep=1)

    def rollback(self, length: int) -> None:
        self.state.cache.rollback(length)


class NativeRunner:
    """The unwrapped model on transformers' own cache and attention: the comparison target of the wrapper's A read
    (reference qwen_wrap.py:489-531). Not a path of this build's kernels."""

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
        T = input_ids.shape[1]
        outs, logits = [], None
        for a in range(0, T, chunk):
            logits = self.forward(input_ids[:, a:a + chunk], logits_to_keep=0 if keep_logits else 1)
            if keep_logits:
                outs.append(logits)
        return torch.cat(outs, dim=1) if keep_logits else logits

    def step(self, token_ids: torch.Tensor) -> torch.Tensor:
        return self.forward(token_ids, logits_to_keep=1)

    def rollback(self, length: int) -> None:
        removed = self.length - int(length)
        if removed < 0:
            raise ValueError("cannot roll forward")
        if removed == 0:
            return
        layers = self.cache.layers
        if all(hasattr(lay, "cumulative_length") and isinstance(lay.cumulative_length, torch.Tensor) for lay in layers):
            for lay in layers:      # static layers: slots beyond `length` fall outside the causal mask
                lay.cumulative_length.fill_(int(length))
        else:
            self.cache.crop(-removed)
        self.length = int(length)


def tiny_qwen3(*, seed: int = 0, layers: int = 2, hidden: int = 64, heads: int = 4, groups: int = 2, head_dim: int = 16,
               intermediate: int = 128, vocab: int = 256, max_positions: int = 2048, dtype=torch.float64):
    """A randomly initialised Qwen3 from a local config (no download). The HIP kernels need head_dim=128 and bf16."""
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
    """K/V [B,G,L,d] a transformers cache holds for one layer (the comparison target of the static cache)."""
    lay = cache.layers[layer]
    return lay.keys, lay.values
