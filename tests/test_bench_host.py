"""bench.py's host side (no GPU): the one-GPU contract, the algorithmic byte counts behind `roofline.achieved`, and
the rocprofv3 counter summaries behind `roofline.traffic` and the matrix-core busy fraction."""
from __future__ import annotations

import csv
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 2
    line = json.loads(res.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def layer_stack(B, G, h, L, rho_k, lists_only=True):
    """A LayerStack's shape attributes without its tensors (the byte counts are arithmetic on them). lists_only: the
    step's list select, where the score kernel stores no score."""
    ls = bench.LayerStack.__new__(bench.LayerStack)
    ls.B, ls.G, ls.h, ls.d, ls.r, ls.L, ls.C = B, G, h, 128, 32, L, L
    ls.lo, ls.hi = 4, L - 64
    ls.M = ls.hi - ls.lo
    ls.k = rho_k
    ls.S = 68 + rho_k
    ls.lists_only = lists_only
    return ls


def test_algorithmic_bytes_follow_the_per_unit_formulas():
    """32K, rho = 1/32 (k = 1024, S = 1092), B = 1, G = 8, h = 2: the per-(b, g) figures of the measurement plan
    (zT columns + fp32 scores; scores + indices; K/V rows + row ids + q + bf16 out; the whole dense read)."""
    ls = layer_stack(1, 8, 2, 32768, 1024, lists_only=False)
    M = 32700
    assert ls.score_bytes() == 8 * (32 * M * 2 + 4 * M + 32 * 2 + (2 * 128 + 128) * 2) + 8 * (2 * 128 * 32 + 32 * 128) * 2
    assert 8 * (32 * M * 2 + 4 * M) == 17_788_800        # the zT read + score write part: 17.79 MB
    assert ls.select_bytes() == 8 * (4 * M + 4 * 1024)
    assert ls.attend_bytes() == 8 * (1092 * 512 + 4 * 1092 + 2 * 128 * 2 * 2)
    assert ls.dense_bytes() == 8 * (32768 * 512 + 2 * 128 * 2 * 2)
    big = layer_stack(16, 8, 4, 32768, 1024, lists_only=False)
    assert big.score_bytes() + big.select_bytes() + big.attend_bytes() == 374_773_760   # stored scores, bench shape
    # the list select's step: no score reaches HBM, so neither the score write nor the select's read is credited
    ls = layer_stack(1, 8, 2, 32768, 1024)
    assert ls.score_bytes() == 8 * (32 * M * 2 + 32 * 2 + (2 * 128 + 128) * 2) + 8 * (2 * 128 * 32 + 32 * 128) * 2
    assert ls.select_bytes() == 8 * 4 * 1024
    big = layer_stack(16, 8, 4, 32768, 1024)
    assert big.score_bytes() + big.select_bytes() + big.attend_bytes() == 374_773_760 - 128 * 8 * M


def test_prefill_score_counts():
    ps = bench.PrefillScore.__new__(bench.PrefillScore)
    ps.B, ps.KG, ps.T, ps.L, ps.nh, ps.r = 1, 8, 8192, 8192, 4, 32
    assert ps.scores() == 8 * 8192 * 8193 // 2 == 268_468_224
    assert ps.algorithmic_bytes() == 4 * ps.scores() + 8 * (8192 * 64 + 8192 * 4 * 128 + 8192 * 16)
    assert ps.flops() == ps.scores() * 4 * (64 + 2)


def write_counters(path, rows):
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for r in rows:
            w.writerow(r)


def test_traffic_summary_scales_each_counter_by_the_copy(tmp_path, capsys):
    copy = "__amd_rocclr_copyBuffer"
    scan = f"void attnlab::{bench.SCAN_KERNEL}<4>(attnlab::ScoreArgs)"
    fetch, write = str(tmp_path / "f"), str(tmp_path / "w")
    # FETCH_SIZE counts half of what moves (the copy reads 256 MiB = 262144 KiB and shows 131072); small set-up copies
    # are ignored
    write_counters(fetch, [{"Kernel_Name": scan, "Counter_Name": "FETCH_SIZE", "Counter_Value": 1000.0}] * 5 +
                   [{"Kernel_Name": copy, "Counter_Name": "FETCH_SIZE", "Counter_Value": 131072.0}] * 5 +
                   [{"Kernel_Name": copy, "Counter_Name": "FETCH_SIZE", "Counter_Value": 4.0}])
    write_counters(write, [{"Kernel_Name": scan, "Counter_Name": "WRITE_SIZE", "Counter_Value": 300.0}] * 5 +
                   [{"Kernel_Name": copy, "Counter_Name": "WRITE_SIZE", "Counter_Value": 262144.0}] * 5)
    assert bench.pmc_summary(fetch, write) == 0
    out = json.loads(capsys.readouterr().out)
    assert out["fetch_scale"] == pytest.approx(2.0) and out["write_scale"] == pytest.approx(1.0)
    assert out["traffic_bytes_per_launch"] == pytest.approx(1000 * 1024 * 2 + 300 * 1024)


def test_mfma_busy_fraction(tmp_path, capsys):
    k = f"void attnlab::{bench.PREFILL_KERNEL}<true, 4, true>(Args)"
    rows = []
    for name, v in (("SQ_VALU_MFMA_BUSY_CYCLES", 1024 * 1000.0), ("GRBM_GUI_ACTIVE", 8 * 4000.0),
                    ("SQ_INSTS_MFMA", 64000.0), ("SQ_INSTS_VALU", 640000.0)):
        rows.append({"Kernel_Name": k, "Counter_Name": name, "Counter_Value": v})
    write_counters(str(tmp_path), rows)
    assert bench.prefill_pmc_summary(str(tmp_path)) == 0
    out = json.loads(capsys.readouterr().out)
    assert out["mfma_busy_frac"] == pytest.approx(0.25)          # 1000 busy of 4000 cycles per SIMD
    assert out["mfma_cycles_per_instruction"] == pytest.approx(16.0)
    assert out["valu_instructions_per_mfma"] == pytest.approx(10.0)


def test_committed_profiles_feed_the_bench_line():
    """The committed score-kernel PMC summary gives the bench line's traffic: at least the algorithmic bytes of one
    B=16, 32K launch as the step runs it (268,378,112: no score stored) and within a few percent of them (the histogram
    atomics and the key lists)."""
    traffic = bench.measured_traffic()
    assert traffic is not None and 268_378_112 <= traffic <= 1.05 * 268_378_112
    assert 0.0 < bench.mfma_busy_from_profile() < 1.0


def test_p0_p1_geometry_matches_the_reference_benches():
    """Legal length N0 + 1, capacity N0 + 128, k from the rho rule: the P1 gate's S = 1076 sits at N0 = 32256
    (p1_attend_kernel.py:32 names S1076; the lengths are p0_score_kernel.py:36's)."""
    L, C, lay, k = bench.p_geometry(32256, 1 / 32)
    assert (L, C) == (32257, 32384)
    assert (lay.candidate_lo, lay.candidate_hi, lay.candidate_count) == (4, 32193, 32189)
    assert lay.fixed_count + k == 1076 and k == 1008
    L, C, lay, k = bench.p_geometry(8192, 1 / 32)
    assert lay.fixed_count + k == 324 and k == 256


def test_cpu_info_and_the_lightning_cpu_leg():
    """The CPU baseline's host facts (the CPUs the all-cores leg uses never exceed what the process may run on) and
    its configs[1] leg, which must compute the lightning score + top-k the oracle defines."""
    import numpy as np
    import torch

    import bench
    from oracle import exact
    info = bench.cpu_info()
    assert 1 <= info["usable_cpus"] <= info["affinity_cpus"] <= info["logical_cpus"]
    g = torch.Generator().manual_seed(3)
    keys, q, w = torch.randn(8, 500, 32, generator=g), torch.randn(8, 4, 32, generator=g), torch.rand(8, 4, generator=g)
    vals, idx = bench._lightning_cpu(torch, keys, q, w, 16)
    s = exact.lightning_scores(keys.double().numpy()[None], q.double().numpy()[None], w.double().numpy()[None], 0, 500)[0]
    np.testing.assert_allclose(vals.numpy(), np.take_along_axis(s, idx.numpy(), -1), rtol=1e-5, atol=1e-5)
    assert np.array_equal(np.sort(idx.numpy(), -1), np.sort(exact.topk(s.astype(np.float32), 16), -1))


def test_topk_picks_the_tiled_kernels_by_row_length_and_count():
    """hip_select.topk's automatic choice (also the configs[1] sweep's): tiled kernels for 32K..256K keys, except rows
    of at most 32K keys when 128 or more of them fill half the chip as one workgroup each."""
    from attention_lab import hip_select
    assert not hip_select.use_tiled(1, 16384)
    assert hip_select.use_tiled(1, 32768) and hip_select.use_tiled(64, 32768)
    assert not hip_select.use_tiled(128, 32768) and not hip_select.use_tiled(256, 32768)
    assert hip_select.use_tiled(256, 65536) and hip_select.use_tiled(512, 262144)
    assert not hip_select.use_tiled(1, 262145)


def test_build_refuses_kernels_with_scratch_memory():
    """build() compiles with the compiler's resource report and fails on any kernel that uses scratch memory (a
    register array or spill placed in memory); the parser reads the report's kernel name and scratch size."""
    import __graft_entry__ as ge
    remarks = "\n".join([
        "x.hip:1:1: remark: Function Name: _ZN7attnlab4goodEv [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:1:1: remark:     VGPRs: 53 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark: Function Name: _ZN7attnlab3badEv [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark:     ScratchSize [bytes/lane]: 152 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert ge.scratch_kernels(remarks) == [("_ZN7attnlab3badEv", 152)]
    assert ge.scratch_kernels("") == []
