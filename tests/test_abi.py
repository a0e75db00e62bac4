"""The C ABI: header, binding and library agree; argument validation runs on the host (no GPU, no compute call)."""
from __future__ import annotations

import math

import ctypes
import re
from pathlib import Path

import pytest

from attention_lab import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "attnlab.h"


def header_symbols():
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:const\s+)?[a-z0-9_]+\*?\s+\*?(attnlab_[a-z0-9_]+)\s*\(", text, flags=re.M))


def header_arity(name):
    text = " ".join(HEADER.read_text().split())
    m = re.search(rf"\b{name}\s*\(([^)]*)\)\s*;", text)
    assert m, name
    args = m.group(1).strip()
    return 0 if args in ("", "void") else len(args.split(","))


def test_header_and_binding_declare_the_same_entry_points():
    syms = header_symbols()
    assert syms == set(_native.SIGNATURES), syms ^ set(_native.SIGNATURES)
    for name, (_, args) in _native.SIGNATURES.items():
        assert header_arity(name) == len(args), f"{name}: header has {header_arity(name)} args, binding {len(args)}"


def test_library_exports_every_declared_symbol(native_lib):
    lib = ctypes.CDLL(_native.LIB_PATH)
    for name in header_symbols():
        assert hasattr(lib, name), f"libattnlab.so does not export {name}"
    assert native_lib.attnlab_abi_version() == _native.ABI_VERSION
    assert native_lib.attnlab_target() == b"gfx950"


def test_invalid_arguments_are_rejected_before_any_launch(native_lib):
    """These calls fail validation on the host; no device pointer is touched and no kernel is launched."""
    with pytest.raises(ValueError, match="k <= M"):
        _native.call("attnlab_topk", None, 10, 1, 10, 11, 0, None, None, 11, None)
    with pytest.raises(ValueError, match="write_col"):
        _native.call("attnlab_score_grouped", 16, 16, 16, 16, 16, None, None, 16, 100, 1, 8, 32, 128, 128, 256, 4, 100,
                     50, 1, None, None)
    with pytest.raises(ValueError, match="index width"):
        _native.call("attnlab_score_grouped", 16, None, 16, 16, 16, None, None, 16, 100, 1, 8, 33, 128, 128, 256, 4, 100,
                     120, 1, None, None)
    with pytest.raises(ValueError, match="h=9"):
        _native.call("attnlab_attend", 16, 16, 128 * 128, 128, 16, 16, 10, 1, 8, 9, 10, 128, 1, 0.1, 16, 1, None, None)
    with pytest.raises(ValueError, match="partitions"):
        _native.call("attnlab_dense_decode", 16, 16, 128 * 128, 128, 16, 1, 8, 2, 10, 128, 0, 0.1, 16, 1, None, None)
    with pytest.raises(ValueError, match="legal"):
        _native.call("attnlab_select_rows", 16, 10, 1, 8, 4, 20, 10, 3, 100, 0, 16, 10, None, None, None, 0, None)
    with pytest.raises(ValueError, match="workspace"):
        _native.call("attnlab_sparse_decode_step", *([16] * 8), 1, 8, 2, 32, 4096, 4, 4032, 4096, 128, 4095, 0.1, 0, 4,
                     None, 256, 10, None, None, 16, None)


def _a(x, n=256):
    return (x + n - 1) // n * n


def select_scratch(R, M, k, order):
    """Select scratch. Rows of at most 8 tiles of 4096 keys: per row the above-threshold bitmap (16-byte aligned), 32
    (above, candidate) count pairs and 32 x 128 candidate entries of 8 bytes; longer rows: two bitmaps of one bit per
    candidate. Score order past k = 8192 adds the radix pass's stage (4 bytes) and two buffers (8 bytes) per pick."""
    words = (M + 31) // 32
    region = R * (_a(words * 4, 16) + 32 * 8 + 4096 * 8) if M <= 32768 else R * 2 * 4 * words
    extra = _a(R * k * 4) + 2 * _a(R * k * 8) if (order == 1 and k > 8192) else 0
    return _a(region) + extra


def test_select_scratch_formula(native_lib):
    for R, M, k, order in ((128, 32704, 1024, 0), (8, 1, 1, 1), (1, 4096, 9000 // 3, 1), (1, 40000, 20000, 1),
                           (2, 40000, 20000, 0), (3, 0, 0, 0), (4, 32768, 32768, 1), (16, 131072, 4096, 1)):
        assert native_lib.attnlab_select_scratch_bytes(R, M, k, order) == select_scratch(R, M, k, order)
    assert native_lib.attnlab_select_scratch_bytes(-1, 5, 1, 0) == -1
    assert native_lib.attnlab_select_scratch_bytes(1, 5, 6, 0) == -1


def list_region(BG, lo, hi, k):
    """The score kernel's per-workgroup key lists: workgroups of 8, 4 or 2 sub-tiles of 512 columns (as many as leave
    256 workgroups), else 1, a list of at least lmin = s + 3 floor(sqrt(s)) + 16 keys for the even share
    s = ceil(k * n / M) of n keys per workgroup and at most cap = min(n, lmin + 192 rounded up to 64) entries of 8
    bytes, and an 8-byte header per workgroup. None where the list select does not apply (M > 32768, more than 128
    workgroups per row, 2 * lmin > n)."""
    M = hi - lo
    if k <= 0 or M <= 0 or M > 32768:
        return 0
    span = ((hi + 7) & ~7) - (lo & ~7)
    blocks = BG * ((span + 511) // 512)
    nsub = 8 if blocks >= 8 * 256 else 4 if blocks >= 4 * 256 else 2 if blocks >= 2 * 256 else 1
    n = 512 * nsub
    tiles = (span + n - 1) // n
    share = (k * n + M - 1) // M
    lmin = share + 3 * math.isqrt(share) + 16
    if tiles > 128 or 2 * lmin > n:
        return 0
    cap = min(n, (lmin + 192 + 63) // 64 * 64)
    return _a(BG * tiles * cap * 8) + _a(BG * tiles * 8)


def test_workspace_size_formula(native_lib):
    def expect(B, G, h, lo, hi, legal, k, P):
        a = lambda x: (x + 255) // 256 * 256  # noqa: E731
        BG, M, S = B * G, hi - lo, lo + (legal - hi) + k
        scores = a(BG * ((M + 3) // 4 * 4) * 4) if k > 0 else 0
        u = a(BG * 32 * 4) if k > 0 else 0
        sel = a(max(select_scratch(BG, M, k, 1), list_region(BG, lo, hi, k))) if k > 0 else 0
        return scores + a(BG * S * 4) + u + sel + (a(BG * P * h * 130 * 4) if P > 1 else 0)
    for args in ((16, 8, 4, 4, 32704, 32768, 1024, 4), (1, 8, 2, 4, 1984, 2048, 64, 1), (2, 8, 2, 60, 60, 60, 0, 8),
                 (16, 8, 2, 4, 32704, 32768, 2048, 1), (16, 8, 2, 4, 32704, 32768, 4096, 1),
                 (1, 8, 2, 4, 32704, 32768, 2048, 1),
                 (1, 8, 2, 4, 32704, 32768, 16384, 1), (4, 8, 2, 4, 300, 364, 32, 1)):
        assert native_lib.attnlab_sparse_decode_workspace(*args) == expect(*args)
    # the lists outgrow the tiled select's scratch at B = 16, 32K, k = 4096, and not at k = 1024
    assert list_region(128, 4, 32704, 4096) > select_scratch(128, 32700, 4096, 1)
    assert 0 < list_region(128, 4, 32704, 1024) < select_scratch(128, 32700, 1024, 1)


def test_list_bytes_formula(native_lib):
    for B, G, lo, hi, k in ((16, 8, 4, 32704, 1024), (1, 8, 4, 32704, 1024), (1, 8, 4, 1984, 64), (2, 8, 4, 300, 32),
                            (1, 8, 4, 32704, 16384), (1, 8, 0, 40000, 100), (4, 8, 60, 60, 0), (16, 8, 4, 16320, 512)):
        assert native_lib.attnlab_list_bytes(B, G, lo, hi, k, 0) == list_region(B * G, lo, hi, k)
        # score order: the list select sorts at most LDS_SORT_K picks
        want = 0 if k > _native.LDS_SORT_K else list_region(B * G, lo, hi, k)
        assert native_lib.attnlab_list_bytes(B, G, lo, hi, k, 1) == want
    assert native_lib.attnlab_list_bytes(1, 8, 4, 32704, 9830, 0) > 0
    assert native_lib.attnlab_list_bytes(1, 8, 4, 32704, 9830, 1) == 0
    assert native_lib.attnlab_list_bytes(0, 8, 0, 10, 1, 0) == -1
    assert native_lib.attnlab_list_bytes(1, 8, 0, 10, 11, 0) == -1
    assert native_lib.attnlab_list_bytes(1, 8, 0, 10, 1, 2) == -1


def test_list_select_refuses_shapes_it_does_not_cover(native_lib):
    with pytest.raises(ValueError, match="does not apply"):   # r = 16: not the one-launch score
        _native.call("attnlab_score_grouped_lists", *([16] * 7), 4096, 1, 8, 16, 4096, 128, 256, 4, 4000, 4095, 100,
                     0, 16, 256, 1 << 20, None)
    with pytest.raises(ValueError, match="score order"):      # score order past the LDS sort, before any launch
        _native.call("attnlab_score_grouped_lists", *([16] * 7), 32768, 1, 8, 32, 32768, 128, 256, 4, 32704, 32767,
                     9830, 1, 16, 256, 1 << 24, None)
    with pytest.raises(ValueError, match="does not apply"):   # M = 40000 > 32768
        _native.call("attnlab_select_lists", 16, 40000, 1, 8, 4, 40004, 40068, 100, 40100, 0, 16, 200, None, 16, 256,
                     1 << 20, None, 0, None, None)
    with pytest.raises(ValueError, match="attnlab_list_bytes"):   # lists too small
        _native.call("attnlab_select_lists", 16, 2000, 1, 8, 4, 2004, 2068, 64, 2100, 0, 16, 200, None, 16, 256, 64,
                     None, 0, None, None)
    with pytest.raises(ValueError, match="without stored scores"):   # no scores: the table and u, position order
        _native.call("attnlab_select_lists", None, 2000, 1, 8, 4, 2004, 2068, 64, 2104, 1, 16, 200, None, 16, 256,
                     1 << 20, 16, 0, 16, None)
    with pytest.raises(ValueError, match="without stored scores"):
        _native.call("attnlab_select_lists", None, 2000, 1, 8, 4, 2004, 2068, 64, 2104, 0, 16, 200, None, 16, 256,
                     1 << 20, None, 0, 16, None)
    assert native_lib.attnlab_sparse_decode_workspace(0, 8, 2, 4, 100, 164, 3, 1) == -1
