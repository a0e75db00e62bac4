"""The measurement-only read probes read exactly the bytes their kernels read.

attnlab_scan_probe (the fused score's load-only twin) and attnlab_gather_probe (the attend's) XOR-fold every loaded
32-bit word into one word per thread. A numpy model of each kernel's grid, lane layout and clamping rules folds the
same words; the sinks must match word for word, so the read ceilings in the committed profiles measure the kernels'
own reads. (q_cat = 0 makes u = 0, so the scan probe's u term adds no bit.)
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from attention_lab import _native as nat

pytestmark = pytest.mark.gpu


def fused_tiling(BG, lo, hi):
    span = ((hi + 7) & ~7) - (lo & ~7)
    blocks512 = BG * ((span + 511) // 512)
    nsub = 8 if blocks512 >= 8 * 256 else 4 if blocks512 >= 4 * 256 else 2 if blocks512 >= 2 * 256 else 1
    return nsub, (span + 512 * nsub - 1) // (512 * nsub)


def scan_model(zw, BG, C, lo, hi):
    """zw: the table as uint32 words [BG * 32, C / 2]. One folded word per thread of every workgroup, indexed by the
    workgroup's XCD-contiguous number (the sink's order)."""
    nsub, tiles = fused_tiling(BG, lo, hi)
    out = np.zeros((BG * tiles, 256), dtype=np.uint32)
    c_last = (hi - 1) & ~7
    lane = np.arange(64)
    for lin in range(BG * tiles):
        bg, tile = divmod(lin, tiles)
        cb0 = (lo & ~7) + tile * 512
        for wave in range(4):
            f = np.zeros(64, dtype=np.uint32)
            for s in range(nsub):
                c0 = np.minimum(cb0 + s * tiles * 512 + lane * 8, c_last)
                for jj in range(8):
                    row = zw[bg * 32 + 8 * wave + jj]
                    for w in range(4):
                        f ^= row[c0 // 2 + w]
            out[lin, 64 * wave:64 * wave + 64] = f
    return out


def test_scan_probe_reads_the_fused_score_columns():
    gpu = torch.device("cuda:0")
    for B, G, C, lo, hi in ((1, 2, 4096 + 64, 4, 4096 - 60), (1, 8, 32768, 4, 32768 - 64), (2, 3, 1000, 0, 993)):
        gen = torch.Generator().manual_seed(C + G)
        zT = torch.randint(-32768, 32768, (B * G, 32, C), generator=gen, dtype=torch.int32).to(torch.int16)
        q_cat = torch.zeros(B * G, 256, dtype=torch.bfloat16)
        wq_t = torch.randn(G, 256, 32, generator=gen).to(torch.bfloat16)
        tiles = fused_tiling(B * G, lo, hi)[1]
        sink = torch.full((B * G * ((hi - lo + 16 + 511) // 512) * 256,), -1, dtype=torch.int32, device=gpu)
        zd, qd, wd = zT.to(gpu), q_cat.to(gpu), wq_t.to(gpu)   # held: the kernel reads them after this line
        nat.call("attnlab_scan_probe", zd.data_ptr(), qd.data_ptr(), wd.data_ptr(), B, G, C, 256, lo, hi,
                 sink.data_ptr(), nat.stream_of(gpu))
        torch.cuda.synchronize()
        n = B * G * tiles
        got = sink.cpu().numpy().view(np.uint32)[:n * 256].reshape(n, 256)
        want = scan_model(zT.numpy().view(np.uint32).reshape(B * G * 32, C // 2), B * G, C, lo, hi)
        assert np.array_equal(got, want), f"B={B} G={G} C={C}: the probe read other words than the score kernel"


def gather_model(kw, vw, rows, BG, S, C, Q, P):
    """kw / vw: the caches as uint32 words [BG, C, 64]; rows [BG, S]. One folded word per thread, indexed by
    the workgroup's XCD-contiguous number."""
    out = np.zeros((BG * Q * P, 256), dtype=np.uint32)
    lane = np.arange(64)
    slot, sub = lane >> 3, lane & 7
    Sp = (S + P - 1) // P
    for lin in range(BG * Q * P):
        bg = lin // (Q * P)
        p = (lin - bg * Q * P) % P
        s_begin, s_end = p * Sp, min(S, p * Sp + Sp)
        for wave in range(4):
            f = np.zeros(64, dtype=np.uint32)
            for c0 in range(s_begin, s_end, 4096):
                clen = min(4096, s_end - c0)
                ng = (clen + 7) // 8
                my_ng = (ng - wave + 3) // 4 if ng > wave else 0
                for j in range(my_ng):
                    e = (wave + 4 * j) * 8 + slot
                    pos = rows[bg, c0 + np.minimum(e, clen - 1)]
                    pos = np.where((e < clen) & (pos >= 0) & (pos < C), pos, 0)
                    for base in (4 * sub, 32 + 4 * sub):   # dims 8 sub and 64 + 8 sub: 16 bytes each
                        for w in range(4):
                            f ^= kw[bg, pos, base + w] ^ vw[bg, pos, base + w]
            out[lin, 64 * wave:64 * wave + 64] = f
    return out


@pytest.mark.parametrize("S,Q,P", [(300, 2, 1), (1092, 1, 4), (37, 1, 8)])
def test_gather_probe_reads_the_attend_rows(S, Q, P):
    gpu = torch.device("cuda:0")
    BG, C = 8, 2048
    gen = torch.Generator().manual_seed(S)
    K = torch.randint(-32768, 32768, (BG, C, 128), generator=gen, dtype=torch.int32).to(torch.int16)
    V = torch.randint(-32768, 32768, (BG, C, 128), generator=gen, dtype=torch.int32).to(torch.int16)
    rows = torch.stack([torch.randperm(C, generator=gen)[:S] for _ in range(BG)]).to(torch.int32)
    rows[0, 5] = C + 3   # outside [0, C): read as row 0
    sink = torch.full((BG * Q * P * 256,), -1, dtype=torch.int32, device=gpu)
    Kd, Vd, Rd = K.to(gpu), V.to(gpu), rows.to(gpu)
    nat.call("attnlab_gather_probe", Kd.data_ptr(), Vd.data_ptr(), C * 128, 128, Rd.data_ptr(), S, 1, BG, S, C, Q, P,
             sink.data_ptr(), nat.stream_of(gpu))
    torch.cuda.synchronize()
    got = sink.cpu().numpy().view(np.uint32).reshape(BG * Q * P, 256)
    want = gather_model(K.numpy().view(np.uint32).reshape(BG, C, 64), V.numpy().view(np.uint32).reshape(BG, C, 64),
                        rows.numpy(), BG, S, C, Q, P)
    assert np.array_equal(got, want), "the gather probe read other words than the attend"
