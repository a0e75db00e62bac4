"""attnlab_sparse_decode_step_noalloc (the step with its state and workspace in the library's own device array) against
attnlab_sparse_decode_step on the same inputs, through the C ABI: row lists and outputs bit for bit, on two calls in a
row, the second smaller (fewer rows, a shorter context, the other row order), and a size past its maximum refused."""
from __future__ import annotations

import math

import pytest
import torch

from attention_lab import _native as nat
from attention_lab.decode import prepare_request
from attention_lab.indexer import GroupedIndexer

pytestmark = pytest.mark.gpu


def inputs(gpu, B, h, C, seed, G=8, r=32):
    gen = torch.Generator().manual_seed(seed)
    t = lambda *s: torch.randn(*s, generator=gen).to(torch.bfloat16).to(gpu)  # noqa: E731
    idx = GroupedIndexer(G, h, 128, r, device=gpu, dtype=torch.bfloat16, seed=seed)
    return dict(q=t(B, G, h, 128), q_cat=t(B, G, h * 128), K=t(B, G, C, 128), V=t(B, G, C, 128), zT=t(B, G, r, C),
                k_new=t(B, G, 128), wq_t=idx.wq_t_scaled.contiguous(), wk=idx.wk.contiguous())


def step(gpu, x, B, h, C, L, rho, order, noalloc, with_rows=True):
    G, r = 8, 32
    req = prepare_request(B, G, C, valid_length=L, query_position=L - 1, rho=rho, device=gpu)
    lo, hi, k, S = req.layout.candidate_lo, req.layout.candidate_hi, req.k, req.selected_count
    P = 4
    zT = x["zT"].clone()
    out = torch.empty(B, G, h, 128, dtype=torch.bfloat16, device=gpu)
    rows = torch.empty(B * G, S, dtype=torch.int32, device=gpu)
    flat = torch.empty(B * G * S, dtype=torch.int64, device=gpu)
    head = [x["q"].data_ptr(), x["q_cat"].data_ptr(), x["K"].data_ptr(), x["V"].data_ptr(), zT.data_ptr(),
            x["wq_t"].data_ptr(), x["wk"].data_ptr(), x["k_new"].data_ptr(), B, G, h, r, C, lo, hi, L, k, L - 1,
            1.0 / math.sqrt(128), order, P]
    stream = nat.stream_of(gpu)
    rp, fp = (rows.data_ptr(), flat.data_ptr()) if with_rows else (None, None)
    if noalloc:
        nat.call("attnlab_sparse_decode_step_noalloc", *head, rp, fp, out.data_ptr(), stream)
    else:
        nbytes = nat.lib().attnlab_sparse_decode_workspace(B, G, h, lo, hi, L, k, P)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
        state = torch.zeros(B * G * nat.SELECT_STATE_WORDS, dtype=torch.int32, device=gpu)
        nat.call("attnlab_sparse_decode_step", *head, state.data_ptr(), ws.data_ptr(), nbytes, rp, fp, out.data_ptr(),
                 stream)
        torch.cuda.synchronize()
        assert int(state.abs().sum()) == 0, "the step left its select state dirty"
    torch.cuda.synchronize()
    return out, rows, flat, zT


@pytest.mark.parametrize("first,second", [((4, 4, 4096 + 64, 4096, 1 / 32, nat.ORDER_SCORE),
                                           (1, 2, 2048 + 64, 2048, 1 / 16, nat.ORDER_POSITION)),
                                          ((2, 2, 32768, 32768, 1 / 32, nat.ORDER_POSITION),
                                           (2, 2, 1000, 900, 1 / 8, nat.ORDER_SCORE))])
def test_no_alloc_step_matches_the_step(gpu, first, second):
    for n, (B, h, C, L, rho, order) in enumerate((first, second)):
        x = inputs(gpu, B, h, C, seed=31 + n)
        want = step(gpu, x, B, h, C, L, rho, order, noalloc=False)
        got = step(gpu, x, B, h, C, L, rho, order, noalloc=True)
        for a, b, name in zip(got, want, ("out", "rows", "flat", "zT")):
            assert torch.equal(a, b), f"call {n + 1}: {name} differs from attnlab_sparse_decode_step"


def test_no_alloc_step_without_rows_matches_the_step(gpu):
    """Without a row list (the step's select-and-attend launch), on the library's own state: two calls in a row, the
    second smaller, each equal to attnlab_sparse_decode_step bit for bit; a third call with rows afterwards still
    matches (the fused launch left the library's state zero)."""
    calls = ((2, 4, 16384 + 64, 16384, 1 / 32, nat.ORDER_POSITION, False),
             (1, 2, 2048 + 64, 2048, 1 / 16, nat.ORDER_POSITION, False),
             (1, 2, 2048 + 64, 2048, 1 / 16, nat.ORDER_POSITION, True))
    for n, (B, h, C, L, rho, order, with_rows) in enumerate(calls):
        x = inputs(gpu, B, h, C, seed=51 + n)
        want = step(gpu, x, B, h, C, L, rho, order, noalloc=False, with_rows=with_rows)
        got = step(gpu, x, B, h, C, L, rho, order, noalloc=True, with_rows=with_rows)
        names = ("out", "rows", "flat", "zT") if with_rows else ("out", "zT")
        for a, b, name in zip((got[0], got[1], got[2], got[3]) if with_rows else (got[0], got[3]),
                              (want[0], want[1], want[2], want[3]) if with_rows else (want[0], want[3]), names):
            assert torch.equal(a, b), f"call {n + 1}: {name} differs from attnlab_sparse_decode_step"


def test_no_alloc_refuses_more_than_it_holds(gpu):
    B, h, C, L = 40, 2, 64, 64        # 320 rows of select state: more than its 256
    x = inputs(gpu, 1, 1, 64, seed=1)
    z = 0
    with pytest.raises(ValueError, match="no-allocation"):
        nat.call("attnlab_sparse_decode_step_noalloc", *([x["q"].data_ptr()] * 8), B, 8, h, 32, C, 4, 4, L, 0, L - 1,
                 0.1, 0, 1, None, None, x["q"].data_ptr(), nat.stream_of(gpu))
    with pytest.raises(ValueError, match="no-allocation"):   # 16 x 8 rows of a 128K context: scores past 32 MiB
        nat.call("attnlab_sparse_decode_step_noalloc", *([x["q"].data_ptr()] * 8), 16, 8, 2, 32, 131072, 4,
                 131072 - 64, 131072, 4096, 131071, 0.1, 0, 1, None, None, x["q"].data_ptr(), nat.stream_of(gpu))
    assert z == 0
