"""ctypes binding of libattnlab.so, the C ABI declared in include/attnlab.h.

torch is imported before the library is opened: torch ships its own HIP runtime under the soname libamdhip64.so.7,
and the dynamic loader then resolves the library's libamdhip64.so.7 dependency to that same runtime, so the kernels
launch on torch's streams and see torch's allocations. There is no fallback path: when the library is missing or
cannot load, every op raises RuntimeError.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_NAME = "libattnlab.so"
# ATTNLAB_LIB names another build of the same library (the host-sanitized debug build); unset, the in-tree one
LIB_PATH = os.environ.get("ATTNLAB_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 9
# select state per (b, g) row: the first-digit histogram of the top-k (2048 bins, top 11 bits of the order-preserving
# score key), 64 super-bin counts of 32 bins each, then 64 arrival counters of the step's attend partitions
# (ATTNLAB_SELECT_STATE_WORDS)
SELECT_STATE_WORDS = 2176

ATTNLAB_OK, ATTNLAB_EINVAL, ATTNLAB_ERUNTIME = 0, 1, 2
LDS_SORT_K = 8192   # ATTNLAB_LDS_SORT_K: score order past this k goes through the select scratch
ORDER_POSITION, ORDER_SCORE = 0, 1
DT_BF16, DT_F16, DT_F32 = 0, 1, 2

_p, _i, _i64, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float

# name -> (restype, argtypes); mirrors include/attnlab.h one to one
SIGNATURES = {
    "attnlab_abi_version": (_i, []),
    "attnlab_last_error": (ctypes.c_char_p, []),
    "attnlab_target": (ctypes.c_char_p, []),
    "attnlab_score_grouped": (_i, [_p] * 8 + [_i64] + [_i] * 10 + [_p, _p]),
    "attnlab_score_prologue": (_i, [_p] * 6 + [_i] * 7 + [_p]),
    "attnlab_project_keys": (_i, [_p, _i64, _i64, _p, _p] + [_i] * 7 + [_p]),
    "attnlab_score_grouped_f32": (_i, [_p] * 8 + [_i64] + [_i] * 9 + [_p, _p]),
    "attnlab_project_keys_f32": (_i, [_p, _i64, _i64, _p, _p] + [_i] * 7 + [_p]),
    "attnlab_score_lightning": (_i, [_p, _i, _p, _p, _p, _i64] + [_i] * 8 + [_p]),
    "attnlab_score_lightning_batched": (_i, [_p, _i, _p, _p, _p, _i64] + [_i] * 10 + [_p]),
    "attnlab_topk": (_i, [_p, _i64] + [_i] * 4 + [_p, _p, _i64, _p]),
    "attnlab_topk_tiled": (_i, [_p, _i64] + [_i] * 4 + [_p, _p, _i64, _p, _p, _i64, _p]),
    "attnlab_select_rows": (_i, [_p, _i64] + [_i] * 8 + [_p, _i64, _p, _p, _p, _i64, _p]),
    "attnlab_select_scratch_bytes": (_i64, [_i] * 4),
    "attnlab_list_bytes": (_i64, [_i] * 6),
    "attnlab_score_grouped_lists": (_i, [_p] * 7 + [_i64] + [_i] * 11 + [_p, _p, _i64, _p]),
    "attnlab_select_lists": (_i, [_p, _i64] + [_i] * 8 + [_p, _i64, _p, _p, _p, _i64, _p, _i, _p, _p]),
    "attnlab_attend": (_i, [_p, _p, _i64, _i, _p, _p, _i64] + [_i] * 6 + [_f, _p, _i, _p, _p]),
    "attnlab_dense_decode": (_i, [_p, _p, _i64, _i, _p] + [_i] * 6 + [_f, _p, _i, _p, _p]),
    "attnlab_attend_paged": (_i, [_p, _p, _i, _i, _p, _i64, _i, _p, _p, _i64] + [_i] * 5 + [_f, _p, _i, _p, _p]),
    "attnlab_prefill_attend": (_i, [_p, _p, _p, _i64, _i, _p] + [_i] * 8 + [_f, _p]),
    "attnlab_prefill_part_bytes": (_i64, [_i] * 5),
    "attnlab_prefill_attend_split": (_i, [_p, _p, _p, _i64, _i, _p] + [_i] * 8 + [_f, _i, _p, _i64, _p]),
    "attnlab_sparse_decode_workspace": (_i64, [_i] * 8),
    "attnlab_sparse_decode_step": (_i, [_p] * 8 + [_i] * 10 + [_f, _i, _i, _p, _p, _i64, _p, _p, _p, _p]),
    "attnlab_sparse_decode_step_f32": (_i, [_p] * 8 + [_i] * 10 + [_f, _i, _i, _p, _p, _i64, _p, _p, _p, _p]),
    "attnlab_sparse_decode_step_noalloc": (_i, [_p] * 8 + [_i] * 10 + [_f, _i, _i, _p, _p, _p, _p]),
    "attnlab_gather_probe": (_i, [_p, _p, _i64, _i, _p, _i64] + [_i] * 6 + [_p, _p]),
    "attnlab_scan_probe": (_i, [_p, _p, _p] + [_i] * 6 + [_p, _p]),
}

_lock = threading.Lock()
_lib = None
_load_error: str | None = None


def _open():
    global _lib, _load_error
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            _load_error = f"{LIB_PATH} is not built (run __graft_entry__.build())"
            raise RuntimeError(_load_error)
        try:
            lib = ctypes.CDLL(LIB_PATH)
        except OSError as e:  # pragma: no cover - depends on the host
            _load_error = f"cannot load {LIB_PATH}: {e}"
            raise RuntimeError(_load_error) from e
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        if lib.attnlab_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {lib.attnlab_abi_version()}, this binding expects {ABI_VERSION}")
        _lib = lib
        return lib


def lib():
    """The loaded library; raises RuntimeError when it is not built or cannot load."""
    return _lib if _lib is not None else _open()


def loadable() -> bool:
    try:
        lib()
        return True
    except RuntimeError:
        return False


def gpu_available() -> bool:
    """A HIP device is visible and the library loads (the counterpart of metal_*.available())."""
    return torch.cuda.is_available() and loadable()


def call(name: str, *args) -> None:
    """Invoke a C-ABI entry point and turn a non-zero status into ValueError / RuntimeError."""
    rc = getattr(lib(), name)(*args)
    if rc != ATTNLAB_OK:
        msg = (lib().attnlab_last_error() or b"").decode(errors="replace")
        if rc == ATTNLAB_EINVAL:
            raise ValueError(f"{name}: {msg}")
        raise RuntimeError(f"{name} failed (status {rc}): {msg}")


def stream_of(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device` (kernels launch where torch would launch)."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


class Workspace:
    """Growable device scratch owned by one op object (split-K partials, intermediate scores, row lists, select
    state).

    Buffers are zero-filled when allocated: the select state (top-k histograms and counters) must start at zero, and
    the kernels leave it zeroed after every call. Two launches that share one Workspace must be ordered on one stream.

    HIP graphs: a captured launch keeps the address of the buffer it was given. A buffer that a larger call replaces is
    therefore never freed here: it is retired but kept alive, so a graph captured before the growth still replays into
    memory nobody else owns (and its select state, left zeroed by every call, stays valid). Growth takes slack
    (a quarter more, at least 1 MiB) so that a decode loop whose sizes creep up step by step reallocates rarely.
    Growing while the current stream is capturing raises RuntimeError: grow it with one eager call of the largest
    shape first. `release_retired()` frees the retired buffers once no graph that used them will replay.
    """

    SLACK_MIN = 1 << 20

    def __init__(self):
        self._bytes: dict = {}
        self._retired: list = []

    def bytes(self, device: torch.device, nbytes: int, tag: str = "main") -> torch.Tensor:
        key = (device, tag)
        buf = self._bytes.get(key)
        nbytes = max(int(nbytes), 256)
        if buf is None or buf.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(f"workspace '{tag}' must grow to {nbytes} bytes during HIP graph capture; run one "
                                   "eager call of this shape before capturing")
            if buf is not None:
                self._retired.append(buf)   # a captured graph may still hold its address
                nbytes = max(nbytes, buf.numel() + max(buf.numel() // 4, self.SLACK_MIN))
            buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)
            self._bytes[key] = buf
        return buf

    def retired_bytes(self) -> int:
        return sum(int(b.numel()) for b in self._retired)

    def release_retired(self) -> None:
        """Free the buffers replaced by growth (only when no captured graph that used them replays again)."""
        self._retired.clear()
