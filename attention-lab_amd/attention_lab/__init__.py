"""attention_lab on MI355X: the sparse-decode hot path of wlvh/attention-lab on hand-written gfx950 HIP kernels.

The import surface mirrors the reference package (src/attention_lab/__init__.py:14-32) so code written against it
switches by putting `attention-lab_amd/` on sys.path instead of `src/`. The Metal modules' counterparts are
`hip_score` (MetalScore) and `hip_attend` (MetalAttend); `hip_select` is the top-k kernel the reference never built.
`dense_reference` / `dense_mask_reference` are the reference's explicit-math comparison targets (float32 torch code in
`reference.py`), exported for the same tests; no read path of this package calls them.
Importing needs only torch; the kernels load from libattnlab.so on first use and every op raises when it is absent.
The Qwen3 wrapper (`qwen_wrap`) needs transformers and is imported explicitly, as in the reference.
"""
__version__ = "0.1.0"
IMPLEMENTATION_STATUS = "mi355x_sparse_decode_hot_path"

from .selection import (FIXED_PREFIX, FIXED_RECENT, SelectionLayout, fixed_budget,  # noqa: E402
                        legal_length, selection_layout)
from .reference import dense_mask_reference, dense_reference  # noqa: E402
from .sparse import flatten_cache, gather_attention, gather_rows, row_offsets, subset_attention  # noqa: E402
from .full import FULL_BACKENDS, full_attention  # noqa: E402
from .indexer import GroupedIndexer, candidate_scores, project_keys, project_queries  # noqa: E402
from .decode import (DecodeRequest, dense_decode_step, gathered_decode_step_kernel, prepare_request,  # noqa: E402
                     select_rows_kernel, select_rows_recent, select_rows_uniform, sparse_decode_step,
                     sparse_decode_step_kernel)

__all__ = [
    "FIXED_PREFIX", "FIXED_RECENT", "SelectionLayout", "fixed_budget", "legal_length", "selection_layout",
    "dense_reference", "dense_mask_reference",
    "flatten_cache", "gather_attention", "gather_rows", "row_offsets", "subset_attention",
    "FULL_BACKENDS", "full_attention",
    "GroupedIndexer", "candidate_scores", "project_keys", "project_queries",
    "DecodeRequest", "dense_decode_step", "gathered_decode_step_kernel", "prepare_request", "select_rows_kernel",
    "select_rows_recent", "select_rows_uniform", "sparse_decode_step", "sparse_decode_step_kernel",
]
