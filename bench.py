#!/usr/bin/env python3
"""Benchmark of the sparse-decode hot path on one MI355X.

Workload (its attention geometry): a Qwen3-8B-shaped stack of 36 layers, each with its own
bf16 K/V cache [16, 8, 32768, 128] and bf16 index table [16, 8, 32, 32768] resident in HBM (~87 GB), 4 query heads
per KV group, one r=32 grouped indexer per layer (seeded as the reference seeds them), rho = 1/32 -> k = 1024 of the
32700 candidates, S = 1092 rows per (b, g). Synthetic data: K, V, index keys, queries ~ N(0, 1).

One step = one decode step of the attention hot path over all 36 layers for the whole batch: per layer, z column
write + u projection + candidate scan, top-k + merge with F, gather-free split-K attention (the D read), captured in a
HIP graph and replayed. `value` = batch x steps / elapsed = tokens/s of that path; the same step with the dense decode
kernel (the A read) is timed beside it. Per-kernel averages come from HIP events around graphs of one kernel type.

`prefill_score` times the batched (prefill) lightning score on the matrix cores beside it: one 8192-token causal
chunk, 8 index key groups, 4 heads of r = 32, fp16 keys (bench.py's PrefillScore).

The CPU baseline runs the reference's own op sequence (matmul, torch.topk, cat, index_select, SDPA; oracle/ref_path)
on the host cores for a bounded sample of layer-steps of the same shapes, and is reported, not targeted.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "attention-lab_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_HBM_GBS = 8000.0
DEFAULT_METRIC = "decode tok/s @32K ctx ρ=1/32; per-layer score+topk+attend µs; HBM GB/s %peak"


def metric_name() -> str:
    try:
        with open(os.path.join(ROOT, "BASELINE.json"), encoding="utf-8") as f:
            return json.load(f)["metric"]
    except (OSError, KeyError, ValueError):
        return DEFAULT_METRIC


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--context", type=int, default=32768)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--groups", type=int, default=8)
    ap.add_argument("--heads-per-group", type=int, default=4)
    ap.add_argument("--index-dim", type=int, default=32)
    ap.add_argument("--rho", type=float, default=1 / 32)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-b1", action="store_true", help="skip the batch-1 per-layer figures")
    ap.add_argument("--no-prefill", action="store_true", help="skip the batched (prefill) lightning score figure")
    ap.add_argument("--kernel-reps", type=int, default=20, help="graph replays per kernel-average measurement")
    ap.add_argument("--pmc-workload", nargs="?", const="scan", choices=("scan", "select"),
                    help="short run for rocprofv3 --pmc passes at the bench shape: 5 launches of one layer's scan "
                         "(scan) or of its score + tiled select pair (select), then 5 plain 256 MiB device copies that "
                         "calibrate the counters; prints one JSON line")
    ap.add_argument("--pmc-table", nargs="+", metavar="DIR",
                    help="per-kernel means of every counter in the rocprofv3 --pmc output directories given (FETCH_SIZE "
                         "and WRITE_SIZE also in bytes, scaled by the 256 MiB calibration copy); no GPU needed")
    ap.add_argument("--sweeps", nargs="?", const="all", choices=("all", "score", "attend"),
                    help="instead of the bench line: the microbenchmark sweeps of BASELINE configs[1] (lightning score "
                         "+ top-k) and configs[2] (gather-free attend vs dense), one JSON line per case")
    ap.add_argument("--c4", action="store_true",
                    help="instead of the bench line: BASELINE configs[3], a random-init Qwen3-1.7B-shaped model read "
                         "through the wrapper: 8192-token prompt, 128 greedy steps on the full read, the same tokens on "
                         "the sparse read (rho = 1/32); per-step logits compared, one JSON line")
    ap.add_argument("--c4-steps", type=int, default=128)
    ap.add_argument("--c4-prompt", type=int, default=8192)
    ap.add_argument("--c5", action="store_true",
                    help="instead of the bench line: BASELINE configs[4], a random-init Qwen3-8B-shaped model read "
                         "through the wrapper at batch 16 x 32K context (uniform random ids): 64 greedy steps on the "
                         "full read, the same tokens on the sparse read (rho = 1/32), eager per-step times; one JSON "
                         "line")
    ap.add_argument("--c5-steps", type=int, default=64)
    ap.add_argument("--c5-context", type=int, default=32768)
    ap.add_argument("--c5-batch", type=int, default=16)
    ap.add_argument("--c5-chunk", type=int, default=2048, help="prefill chunk of the configs[4] run")
    ap.add_argument("--p0", action="store_true",
                    help="instead of the bench line: the reference's P0 score bench (bench/p0_score_kernel.py) on the "
                         "HIP score ops: batch 1, G=8, h=2, 28 rotating layers per length; PyTorch chain / score-only "
                         "vs fused one- and two-launch; numerics and the stop gate; one JSON line per length + summary")
    ap.add_argument("--p1", action="store_true",
                    help="instead of the bench line: the reference's P1 attend bench (bench/p1_attend_kernel.py) on "
                         "the HIP attend: index_select + subset attention vs the gather-free attend at P = 1, 2, 4, 8; "
                         "numerics and the stop gate; one JSON line per length + summary")
    ap.add_argument("--f32-workload", action="store_true",
                    help="instead of the bench line: the fused step over float32 index tables (a trained bank's "
                         "dtype) at the bench shape, 8 rotating layers, graph-timed, with the bf16 step beside it; "
                         "one JSON line (also the command profiled for the fp32 kernels)")
    ap.add_argument("--scan-ceiling", action="store_true",
                    help="instead of the bench line: the fused score kernel against its read probe (attnlab_scan_probe)")
    ap.add_argument("--gather-ceiling", action="store_true",
                    help="instead of the bench line: the attend against a gather-only probe over the step's own row "
                         "lists (every layer of a 36-layer stack, rows from the step itself), at B=16 h=4 and B=1 h=2, "
                         "graph-timed per layer; one JSON line")
    ap.add_argument("--p-lengths", type=int, nargs="+", default=[8192, 16384, 32256], help="N0 of --p0 / --p1")
    ap.add_argument("--p-layers", type=int, default=28, help="rotating layers of --p0 / --p1")
    ap.add_argument("--prefill-workload", action="store_true",
                    help="short run for rocprofv3: 5 launches of the batched (prefill) lightning score at its bench "
                         "shape; prints one JSON line")
    ap.add_argument("--prefill-attend-workload", action="store_true",
                    help="causal prefill attention (attnlab_prefill_attend) at a whole 8K prompt (h = 2, 4), a 1K "
                         "chunk after a 7K history and B=16 x 2K; prints one JSON line")
    ap.add_argument("--index-build-workload", action="store_true",
                    help="instead of the bench line: the bulk index-table build (project_keys, bf16 and float32) "
                         "at B=16, G=8, T=32768, d=128, r=32, 10 HIP-event-timed launches each; one JSON line (also "
                         "the command profiled for these kernels)")
    ap.add_argument("--prefill-pmc-summary", metavar="DIR",
                    help="summarise a rocprofv3 --pmc pass of --prefill-workload (SQ_VALU_MFMA_BUSY_CYCLES, "
                         "GRBM_GUI_ACTIVE, SQ_INSTS_MFMA, SQ_INSTS_VALU) into the matrix-core busy fraction")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarise the counter_collection.csv files of a FETCH_SIZE pass and a WRITE_SIZE pass of "
                         "--pmc-workload into HBM bytes per scan launch (no GPU needed)")
    return ap.parse_args()


PMC_COPY_BYTES = 256 << 20
PREFILL_PROFILE = os.path.join(ROOT, "profiles", "lightning_batched_kg8_t8192_pmc.md")
PREFILL_KERNEL = "lightning_batched"
PEAK_MFMA_F16_TFLOPS = 2500.0   # dense fp16/bf16 matrix-core peak of MI355X
MI355X_SIMDS, MI355X_XCDS = 256 * 4, 8
PMC_PROFILE = os.path.join(ROOT, "profiles", "score_scan_fused_b16_l32k_pmc.md")
SCAN_KERNEL = "score_scan_fused"


def pmc_workload(torch, dev, args):
    ls = LayerStack(torch, dev, batch=args.batch, groups=args.groups, hpg=args.heads_per_group, context=args.context,
                    layers=1, r=args.index_dim, rho=args.rho, seed=args.seed)
    fns = launchers(ls, torch)
    for _ in range(5):
        if args.pmc_workload == "select":
            fns["score_select"](0)
        else:
            fns["score"](0)
    src = torch.ones(PMC_COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_workload": f"{'score + select' if args.pmc_workload == 'select' else SCAN_KERNEL} x5 then "
                                      f"256 MiB copy x5", "select_algorithmic_bytes": ls.select_bytes(),
                      "scores_bytes": 0 if ls.lists_only else ls.B * ls.G * 4 * ls.M,
                      "scan_algorithmic_bytes": ls.score_bytes(),
                      "scan_read_bytes": ls.score_bytes() - ls.B * ls.G * ls.score_write_bytes(),
                      "scan_write_bytes": ls.B * ls.G * ls.score_write_bytes(),
                      "copy_bytes_each_way": PMC_COPY_BYTES}))
    return 0


def _counter_means(directory, counter):
    """Mean counter value per dispatch for the scan kernel and for the calibration copy (torch's copy_ of 256 MiB runs
    as the runtime's __amd_rocclr_copyBuffer kernel; its small set-up copies are told apart by the counter value)."""
    import csv
    import glob
    files = glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {directory}")
    vals = {"scan": [], "copy": []}
    with open(files[0], newline="") as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") != counter:
                continue
            name = row.get("Kernel_Name", "")
            if SCAN_KERNEL in name:
                vals["scan"].append(float(row["Counter_Value"]))
            elif "copyBuffer" in name:
                vals["copy"].append(float(row["Counter_Value"]))
    big = max(vals["copy"], default=0.0)
    vals["copy"] = [v for v in vals["copy"] if v >= 0.5 * big]
    if not vals["scan"] or not vals["copy"]:
        raise SystemExit(f"{counter}: found {len(vals['scan'])} scan and {len(vals['copy'])} copy dispatches")
    return {k: sum(v) / len(v) for k, v in vals.items()}, {k: len(v) for k, v in vals.items()}


def pmc_summary(fetch_dir, write_dir):
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of the scan, each scaled by bytes / counter of the 256 MiB copy."""
    fetch, nf = _counter_means(fetch_dir, "FETCH_SIZE")
    write, nw = _counter_means(write_dir, "WRITE_SIZE")
    f_scale = PMC_COPY_BYTES / (fetch["copy"] * 1024)
    w_scale = PMC_COPY_BYTES / (write["copy"] * 1024)
    read_b = fetch["scan"] * 1024 * f_scale
    write_b = write["scan"] * 1024 * w_scale
    out = {"fetch_kib_scan": fetch["scan"], "fetch_kib_copy": fetch["copy"], "fetch_scale": f_scale,
           "write_kib_scan": write["scan"], "write_kib_copy": write["copy"], "write_scale": w_scale,
           "dispatches": {"fetch": nf, "write": nw}, "traffic_read_bytes": read_b, "traffic_write_bytes": write_b,
           "traffic_bytes_per_launch": read_b + write_b}
    print(json.dumps(out, indent=1))
    return 0


def pmc_table(dirs):
    """Mean value per dispatch of every counter, per kernel (names shortened), over the counter_collection.csv files of
    the given rocprofv3 --pmc directories; FETCH_SIZE / WRITE_SIZE also as bytes, scaled by the 256 MiB copy."""
    import csv
    import glob
    import re
    sums: dict = {}
    for d in dirs:
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(path, newline="") as f:
                for row in csv.DictReader(f):
                    name = row.get("Kernel_Name", "")
                    short = re.sub(r"^void |\(.*$|<.*$|attnlab::", "", name)
                    key = (short, row["Counter_Name"])
                    sums.setdefault(key, []).append(float(row["Counter_Value"]))
    copy = {c: max(v) for (k, c), v in sums.items() if "copyBuffer" in k}
    table: dict = {}
    for (k, c), v in sorted(sums.items()):
        if "copyBuffer" in k:
            continue
        if len(v) < 5:   # the workload's kernels run 5 times; torch's set-up kernels fewer
            continue
        mean = sum(v) / len(v)
        ent = table.setdefault(k, {})
        ent[c] = mean
        if c in copy and c in ("FETCH_SIZE", "WRITE_SIZE"):
            ent[c + "_bytes"] = mean * PMC_COPY_BYTES / copy[c]
        ent["dispatches_" + c] = len(v)
    print(json.dumps({"kernels": table, "copy_reading": copy}, indent=1))
    return 0


def measured_traffic():
    """HBM bytes per scan launch recorded by the committed rocprofv3 --pmc summary, or None."""
    import re
    try:
        with open(PMC_PROFILE, encoding="utf-8") as f:
            m = re.search(r"traffic_bytes_per_launch:\s*([0-9.]+)", f.read())
        return float(m.group(1)) if m else None
    except OSError:
        return None


# ---------------------------------------------------------------------------------------------------------------------
# workload
# ---------------------------------------------------------------------------------------------------------------------
class LayerStack:
    """Per-layer caches, index tables, weights and queries of one decode step, plus preallocated outputs."""

    def __init__(self, torch, dev, *, batch, groups, hpg, context, layers, r, rho, seed):
        from attention_lab.decode import prepare_request
        from attention_lab.indexer import GroupedIndexer
        self.B, self.G, self.h, self.d, self.r, self.L, self.n = batch, groups, hpg, 128, r, context, layers
        self.C = context
        B, G, h, d, C = self.B, self.G, self.h, self.d, self.C
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        bf = torch.bfloat16
        self.K, self.V, self.zT, self.q, self.q_cat, self.k_new, self.wq_t, self.wk = ([] for _ in range(8))
        for l in range(layers):
            self.K.append(torch.randn(B, G, C, d, device=dev, dtype=bf, generator=gen))
            self.V.append(torch.randn(B, G, C, d, device=dev, dtype=bf, generator=gen))
            self.zT.append(torch.randn(B, G, r, C, device=dev, dtype=bf, generator=gen))
            self.q.append(torch.randn(B, G, h, d, device=dev, dtype=bf, generator=gen))
            self.q_cat.append(torch.randn(B, G, h * d, device=dev, dtype=bf, generator=gen))
            self.k_new.append(torch.randn(B, G, d, device=dev, dtype=bf, generator=gen))
            idx = GroupedIndexer(G, h, d, r, device=dev, dtype=bf, seed=seed * 1000 + l)
            self.wq_t.append(idx.wq_t_scaled)
            self.wk.append(idx.wk)
        req = prepare_request(B, G, C, valid_length=context, query_position=context - 1, rho=rho, device=dev)
        self.req = req
        self.lo, self.hi, self.k = req.layout.candidate_lo, req.layout.candidate_hi, req.k
        self.S, self.write_col, self.k0 = req.selected_count, req.write_col, req.k0
        self.M = self.hi - self.lo
        self.out = [torch.empty(B, G, h, d, device=dev, dtype=bf) for _ in range(layers)]
        self.dense_out = [torch.empty(B, G, h, d, device=dev, dtype=bf) for _ in range(layers)]
        self.scores = torch.empty(B, G, (self.M + 3) // 4 * 4, device=dev, dtype=torch.float32)
        self.rows = torch.empty(B, G, self.S, device=dev, dtype=torch.int32)
        # the step (position order) stores no score where the list select applies: the score kernel writes key lists
        # only and the select recomputes the rare tile it needs from the table; elsewhere (tiled select) it stores them
        from attention_lab import _native as nat
        self.lists_only = nat.lib().attnlab_list_bytes(B, G, self.lo, self.hi, self.k, nat.ORDER_POSITION) > 0

    # -- algorithmic bytes per launch (per layer) --
    def score_write_bytes(self):
        """Per (b, g): the fp32 scores (only where the step stores them) and the bf16 z column."""
        return (0 if self.lists_only else 4 * self.M) + 2 * self.r

    def score_bytes(self):
        """The score kernel: index-table columns [lo, hi) read per (b, g), the fp32 scores written where the step stores
        them (not with the list select, whose step never puts its scores in HBM), q_cat, k_new and the z column per
        (b, g), and the projection weights per group."""
        B, G, h, d, r, M = self.B, self.G, self.h, self.d, self.r, self.M
        return B * G * (r * M * 2 + self.score_write_bytes() + (h * d + d) * 2) + G * (h * d * r + r * d) * 2

    def select_bytes(self):
        """Per (b, g): the k picks written, plus the scores read where the step stores them."""
        return self.B * self.G * ((0 if self.lists_only else 4 * self.M) + 4 * self.k)

    def attend_bytes(self):
        B, G, h, d, S = self.B, self.G, self.h, self.d, self.S
        return B * G * (S * d * 2 * 2 + 4 * S + h * d * 2 + h * d * 2)

    def dense_bytes(self):
        B, G, h, d = self.B, self.G, self.h, self.d
        return B * G * (self.L * d * 2 * 2 + h * d * 2 * 2)


def launchers(ls, torch):
    """Callables that launch one layer's work on the current stream (no allocation, no sync)."""
    from attention_lab import _native as nat
    from attention_lab import hip_attend
    lib = nat.lib()
    dev = ls.K[0].device
    B, G, h, d, r, C = ls.B, ls.G, ls.h, ls.d, ls.r, ls.C
    P = hip_attend.sparse_partitions(B * G, ls.S, h, merged=True)   # the step: partials merged in-kernel
    Pa = hip_attend.sparse_partitions(B * G, ls.S, h)                # the standalone attend: the combine kernel
    Pd = hip_attend.dense_partitions(B * G, ls.L)
    ws_bytes = lib.attnlab_sparse_decode_workspace(B, G, h, ls.lo, ls.hi, ls.L, ls.k, P)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    part = torch.empty(B * G * max(P, Pa, Pd) * h * 130, dtype=torch.float32, device=dev)
    # select state (top-k histograms and counters): zero once; each score/select pair leaves it zeroed
    step_hist = torch.zeros(B * G * nat.SELECT_STATE_WORDS, dtype=torch.int32, device=dev)
    hist = torch.zeros(B * G * nat.SELECT_STATE_WORDS, dtype=torch.int32, device=dev)
    sel_bytes = lib.attnlab_select_scratch_bytes(B * G, ls.M, ls.k, nat.ORDER_POSITION)
    sel_scratch = torch.empty(sel_bytes, dtype=torch.uint8, device=dev)
    # the list select (what the fused step runs where it applies): the score kernel's key lists
    list_bytes = lib.attnlab_list_bytes(B, G, ls.lo, ls.hi, ls.k, nat.ORDER_POSITION)
    lists = torch.empty(max(list_bytes, 256), dtype=torch.uint8, device=dev)
    u_buf = torch.zeros(B * G * r, dtype=torch.float32, device=dev)
    scale = 1.0 / math.sqrt(d)

    def stream():
        return torch.cuda.current_stream(dev).cuda_stream

    def sparse(l):
        nat.call("attnlab_sparse_decode_step", ls.q[l].data_ptr(), ls.q_cat[l].data_ptr(), ls.K[l].data_ptr(),
                 ls.V[l].data_ptr(), ls.zT[l].data_ptr(), ls.wq_t[l].data_ptr(), ls.wk[l].data_ptr(),
                 ls.k_new[l].data_ptr(), B, G, h, r, C, ls.lo, ls.hi, ls.L, ls.k, ls.write_col, scale,
                 nat.ORDER_POSITION, P, step_hist.data_ptr(), ws.data_ptr(), ws_bytes, None, None,
                 ls.out[l].data_ptr(), stream())

    def dense(l):
        nat.call("attnlab_dense_decode", ls.K[l].data_ptr(), ls.V[l].data_ptr(), C * d, d, ls.q[l].data_ptr(), B, G,
                 h, ls.L, C, Pd, scale, ls.dense_out[l].data_ptr(), 1, part.data_ptr(), stream())

    def score(l):   # u, z column, scan (and the key lists) in one launch, as in the fused step: the dominant kernel
        if list_bytes > 0:   # key lists only, no score stored (the step's position order)
            nat.call("attnlab_score_grouped_lists", ls.zT[l].data_ptr(), ls.k_new[l].data_ptr(), ls.wk[l].data_ptr(),
                     ls.q_cat[l].data_ptr(), ls.wq_t[l].data_ptr(), u_buf.data_ptr(), None, ls.scores.shape[2], B, G,
                     r, C, d, h * d, ls.lo, ls.hi, ls.write_col, ls.k, nat.ORDER_POSITION, hist.data_ptr(),
                     lists.data_ptr(), list_bytes, stream())
            return
        nat.call("attnlab_score_grouped", ls.zT[l].data_ptr(), ls.k_new[l].data_ptr(), ls.wk[l].data_ptr(),
                 ls.q_cat[l].data_ptr(), ls.wq_t[l].data_ptr(), None, u_buf.data_ptr(), ls.scores.data_ptr(),
                 ls.scores.shape[2], B, G, r, C, d, h * d, ls.lo, ls.hi, ls.write_col, 1, hist.data_ptr(), stream())

    def select(l):
        if list_bytes > 0:   # from the lists; a tile whose list is incomplete is recomputed from the table and u
            nat.call("attnlab_select_lists", None, ls.scores.shape[2], B, G, ls.lo, ls.hi, ls.L, ls.k, C,
                     nat.ORDER_POSITION, ls.rows.data_ptr(), ls.S, None, hist.data_ptr(), lists.data_ptr(),
                     list_bytes, ls.zT[l].data_ptr(), nat.DT_BF16, u_buf.data_ptr(), stream())
            return
        nat.call("attnlab_select_rows", ls.scores.data_ptr(), ls.scores.shape[2], B, G, ls.lo, ls.hi, ls.L, ls.k, C,
                 nat.ORDER_POSITION, ls.rows.data_ptr(), ls.S, None, hist.data_ptr(), sel_scratch.data_ptr(),
                 sel_bytes, stream())

    def score_select(l):
        score(l)
        select(l)

    def attend(l):   # the standalone attend (split-K partials merged by the combine kernel)
        nat.call("attnlab_attend", ls.K[l].data_ptr(), ls.V[l].data_ptr(), C * d, d, ls.q[l].data_ptr(),
                 ls.rows.data_ptr(), ls.S, B, G, h, ls.S, C, Pa, scale, ls.out[l].data_ptr(), 1, part.data_ptr(),
                 stream())

    return {"sparse": sparse, "dense": dense, "score": score, "select": select, "attend": attend,
            "score_select": score_select, "hist": hist, "partitions": P, "attend_partitions": Pa,
            "dense_partitions": Pd,
            "select_kernels": "select_attend (fused with the attend)" if list_bytes > 0
                              else "select_classify_compact + select_resolve_compact",
            "_keep": (ws, part, step_hist, u_buf, sel_scratch, lists)}


def kernel_breakdown(torch, fns, ls, reps):
    """Per-layer us of each stage of the fused step, from graphs of one launch per layer on consistent data, each
    stage in forward and reverse layer order (median, p95, conservative): score (u, z column, scan and, where the list
    select applies, its key lists: one kernel), select_attend = step - score (the step's second launch where the list
    select applies: every attend workgroup selects its row and attends its partition, merging split-K partials
    in-kernel), select = (score + select) - score (the standalone select_lists launch; it consumes and clears the
    histogram the scan builds; score-only graphs leave it dirty, so it is zeroed before the pair), attend = step -
    (score + select) (what the fused launch costs beyond a standalone select), and attend_standalone, attnlab_attend
    with the combine kernel. The flat figures are the conservative medians; `mean` holds the forward-order means (the
    kernel-trace averages compare with these)."""
    n = ls.n
    score = ordered_stats(torch, fns["score"], n, reps, 3, per=n)
    fns["hist"].zero_()
    torch.cuda.synchronize()
    pair = ordered_stats(torch, fns["score_select"], n, reps, 3, per=n)
    step = ordered_stats(torch, fns["sparse"], n, reps, 3, per=n)
    standalone = ordered_stats(torch, fns["attend"], n, reps, 3, per=n)
    diff = lambda a, b: {o: {k: a[o][k] - b[o][k] for k in ("median_us", "mean_us")} for o in ("forward", "reverse")}
    select, attend, fused = diff(pair, score), diff(step, pair), diff(step, score)
    for x in (select, attend, fused):
        x["conservative_us"] = max(x["forward"]["median_us"], x["reverse"]["median_us"])
    return {"score": score["conservative_us"], "select_attend": fused["conservative_us"],
            "select": select["conservative_us"], "attend": attend["conservative_us"],
            "attend_standalone": standalone["conservative_us"],
            "mean": {"score": score["forward"]["mean_us"], "select_attend": fused["forward"]["mean_us"],
                     "select": select["forward"]["mean_us"], "attend": attend["forward"]["mean_us"]},
            "orders": {"score": score, "score_select": pair, "step": step, "select_attend": fused, "select": select,
                       "attend": attend, "attend_standalone": standalone}}


def capture(torch, fn, layers, reverse=False):
    """A HIP graph that runs fn(l) for every layer, in order 0..layers-1 or, with reverse, layers-1..0."""
    order = range(layers - 1, -1, -1) if reverse else range(layers)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for l in order:
            fn(l)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for l in order:
            fn(l)
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, reps, warmup):
    return replay_stats(torch, g, reps, warmup)["mean_ms"]


def replay_stats(torch, g, reps, warmup):
    """Replays of one graph timed one by one with HIP events on the current stream (an event pair per replay, no sync
    in between): mean, median and p95 in ms per replay, and the samples."""
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    ev[0].record()
    for i in range(reps):
        g.replay()
        ev[i + 1].record()
    torch.cuda.synchronize()
    ms = [ev[i].elapsed_time(ev[i + 1]) for i in range(reps)]
    srt = sorted(ms)
    return {"mean_ms": ev[0].elapsed_time(ev[reps]) / reps, "median_ms": statistics.median(ms),
            "p95_ms": srt[min(reps - 1, int(math.ceil(0.95 * reps)) - 1)], "samples_ms": ms}


def ordered_stats(torch, fn, layers, reps, warmup, per=1.0):
    """The reference's protocol (bench/p0_score_kernel.py:97-110, 203-204): fn over every layer captured once in
    forward and once in reverse layer order, each timed replay by replay; median and p95 per order and the conservative
    figure, the slower order's median. Values are per replay divided by `per` (per layer: the layer count), in us."""
    out = {}
    for name, rev in (("forward", False), ("reverse", True)):
        st = replay_stats(torch, capture(torch, fn, layers, reverse=rev), reps, warmup)
        out[name] = {"median_us": st["median_ms"] * 1e3 / per, "p95_us": st["p95_ms"] * 1e3 / per,
                     "mean_us": st["mean_ms"] * 1e3 / per}
    out["conservative_us"] = max(out["forward"]["median_us"], out["reverse"]["median_us"])
    return out


# ---------------------------------------------------------------------------------------------------------------------
# batched (prefill) lightning score on the matrix cores
# ---------------------------------------------------------------------------------------------------------------------
class PrefillScore:
    """A prefill chunk of the lightning indexer: T = L = 8192 queries (the C4 prompt length) against their causal
    prefixes, 8 index key groups (one per KV group), 4 index heads of r = 32, fp16 keys ~ N(0, 1/32), fp32 queries ~
    N(0, 1), weights ~ U(0, 1), ReLU; fp32 scores of the causal triangle written to [B, KG, T, L]."""

    def __init__(self, torch, dev, *, batch=1, groups=8, tokens=8192, heads=4, seed=0):
        self.B, self.KG, self.T, self.L, self.nh, self.r = batch, groups, tokens, tokens, heads, 32
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        self.keys = (torch.randn(batch, groups, tokens, 32, device=dev, generator=gen) / 32 ** 0.5).to(torch.float16)
        self.q = torch.randn(batch, groups, tokens, heads, 32, device=dev, generator=gen)
        self.w = torch.rand(batch, groups, tokens, heads, device=dev, generator=gen)
        self.out = torch.empty(batch, groups, tokens, tokens, device=dev)

    def launch(self):
        from attention_lab import hip_score
        hip_score.score_lightning_batched(self.keys, self.q, self.w, 0, self.L, q_pos0=0, out=self.out)

    def scores(self):
        return self.B * self.KG * self.T * (self.T + 1) // 2

    def algorithmic_bytes(self):
        """Scores written (4 B each) plus keys, queries and weights read once."""
        B, KG, T, L, nh, r = self.B, self.KG, self.T, self.L, self.nh, self.r
        return 4 * self.scores() + B * KG * (L * r * 2 + T * nh * r * 4 + T * nh * 4)

    def flops(self):
        """Per score: nh dot products of r (2 r flops each), ReLU and the weighted head sum (2 flops per head)."""
        return self.scores() * self.nh * (2 * self.r + 2)


def mfma_busy_from_profile():
    """Matrix-core busy fraction of the batched score recorded by the committed rocprofv3 --pmc summary, or None."""
    import re
    try:
        with open(PREFILL_PROFILE, encoding="utf-8") as f:
            m = re.search(r"mfma_busy_frac:\s*([0-9.]+)", f.read())
        return float(m.group(1)) if m else None
    except OSError:
        return None


def prefill_pmc_summary(directory):
    import csv
    import glob
    files = glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {directory}")
    acc = {}
    for path in files:
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                if PREFILL_KERNEL in row["Kernel_Name"]:
                    acc.setdefault(row["Counter_Name"], []).append(float(row["Counter_Value"]))
    mean = {k: sum(v) / len(v) for k, v in acc.items()}
    busy, gui = mean["SQ_VALU_MFMA_BUSY_CYCLES"], mean["GRBM_GUI_ACTIVE"]
    out = {"dispatches": len(acc["GRBM_GUI_ACTIVE"]), "counters_mean_per_dispatch": mean,
           "cycles_per_xcd": gui / MI355X_XCDS,
           "mfma_busy_frac": busy / MI355X_SIMDS / (gui / MI355X_XCDS),
           "mfma_cycles_per_instruction": busy / mean["SQ_INSTS_MFMA"],
           "valu_instructions_per_mfma": mean["SQ_INSTS_VALU"] / mean["SQ_INSTS_MFMA"]}
    print(json.dumps(out, indent=1))
    return 0


def prefill_workload(torch, dev):
    ps = PrefillScore(torch, dev)
    for _ in range(5):
        ps.launch()
    torch.cuda.synchronize()
    print(json.dumps({"prefill_workload": f"{PREFILL_KERNEL} x5", "scores": ps.scores(),
                      "algorithmic_bytes": ps.algorithmic_bytes(), "flops": ps.flops()}))
    return 0


def index_build_workload(torch, dev, reps=10, B=16, G=8, T=32768, d=128, r=32):
    """The prefill's bulk index-table build, zT[b, g, :, t] = wk[g] . k_pre[b, g, t] for a whole 32K context
    (qwen_wrap.py:320-324 builds it per layer from the prompt's pre-RoPE keys), in bf16 (project_keys_mfma) and in
    float32 (project_keys_f32_mfma, a trained bank's dtype). Algorithmic bytes per position: d keys read and r table
    entries written."""
    from attention_lab import _native as nat
    stream = torch.cuda.current_stream(dev).cuda_stream
    out = {"index_build_workload": f"B={B}, G={G}, T={T}, d={d}, r={r}", "launches": reps}
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    for name, dtype, fn in (("bf16", torch.bfloat16, "attnlab_project_keys"),
                            ("f32", torch.float32, "attnlab_project_keys_f32")):
        k_pre = torch.randn(B, G, T, d, device=dev, generator=gen).to(dtype)
        wk = (torch.randn(G, r, d, device=dev, generator=gen) * 0.05).to(dtype)
        zT = torch.empty(B, G, r, T, device=dev, dtype=dtype)

        def launch():
            nat.call(fn, k_pre.data_ptr(), T * d, d, wk.data_ptr(), zT.data_ptr(), B, G, T, r, d, T, 0, stream)
        launch()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()   # torch's current stream, the stream the kernels launch on
        for _ in range(reps):
            launch()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        nbytes = B * G * T * (d + r) * k_pre.element_size()
        out[name] = {"avg_launch_us": us, "algorithmic_bytes": nbytes, "gbs": nbytes / us / 1e3,
                     "hbm_frac": nbytes / us / 1e3 / PEAK_HBM_GBS}
        del k_pre, wk, zT
        torch.cuda.empty_cache()
    print(json.dumps(out))
    return 0


PREFILL_ATTEND_SHAPES = (   # (B, G, h, T, q_pos0, legal): a whole causal prompt, a chunk after a history, a batch
    (1, 8, 2, 8192, 0, 8192), (1, 8, 4, 8192, 0, 8192), (1, 8, 2, 1024, 7168, 8192), (16, 8, 2, 2048, 0, 2048))


def prefill_attend_workload(torch, dev, reps=10, rounds=5):
    """Causal prefill attention (attnlab_prefill_attend, the full read of full.py:17-44 for a chunk of consecutive
    queries): per shape, 0.3 s of untimed launches, then `rounds` timed runs of `reps` back-to-back launches after two
    untimed ones (HIP events on the launching stream), the median run per launch. Algorithmic flops: 4 d per (query, head, visible key): the two
    products of every score."""
    from attention_lab import _native as nat
    from attention_lab import hip_attend
    stream = torch.cuda.current_stream(dev).cuda_stream
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    out = {"prefill_attend_workload": "causal, d=128, bf16, scale 1/sqrt(d); key splits by hip_attend.prefill_splits "
                                      "(the split read's merge kernel included in the time)", "launches_per_run": reps}
    for (B, G, h, T, p0, legal) in PREFILL_ATTEND_SHAPES:
        C, d = legal, 128
        q = torch.randn(B, G, h, T, d, device=dev, dtype=torch.bfloat16, generator=gen)
        K = torch.randn(B, G, C, d, device=dev, dtype=torch.bfloat16, generator=gen)
        V = torch.randn(B, G, C, d, device=dev, dtype=torch.bfloat16, generator=gen)
        o = torch.empty_like(q)
        splits = hip_attend.prefill_splits(B, G, h, T, p0, legal)   # the wrapper's rule (full_attention, T > 1)
        part = torch.empty(max(nat.lib().attnlab_prefill_part_bytes(B, G, h, T, splits), 16) // 4, device=dev)

        def launch():
            nat.call("attnlab_prefill_attend_split", q.data_ptr(), K.data_ptr(), V.data_ptr(), C * d, d, o.data_ptr(),
                     B, G, h, T, d, p0, legal, C, 1.0 / math.sqrt(d), splits, part.data_ptr(), part.numel() * 4, stream)
        t_warm = time.perf_counter()   # the clocks settle over the first tens of milliseconds of launches
        while time.perf_counter() - t_warm < 0.3:
            for _ in range(reps):
                launch()
            torch.cuda.synchronize()
        runs = []
        for _ in range(rounds):
            for _ in range(2):
                launch()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                launch()
            e1.record()
            torch.cuda.synchronize()
            runs.append(e0.elapsed_time(e1) * 1e3 / reps)
        us = statistics.median(runs)
        flops = B * G * h * sum(min(legal, p0 + t + 1) for t in range(T)) * 4 * d
        out[f"B{B}_G{G}_h{h}_T{T}_after{p0}"] = {"avg_launch_us": us, "runs_us": runs, "flops": flops, "splits": splits,
                                                  "tflops": flops / us / 1e6,
                                                  "mfma_frac_of_peak": flops / us / 1e6 / PEAK_MFMA_F16_TFLOPS}
        print(f"[prefill_attend] B={B} G={G} h={h} T={T} after {p0} (splits {splits}): {us:.1f} us, "
              f"{flops / us / 1e6:.0f} TFLOP/s",
              file=sys.stderr, flush=True)
        del q, K, V, o, part
        torch.cuda.empty_cache()
    print(json.dumps(out))
    return 0


def run_prefill_score(torch, dev, reps=10):
    ps = PrefillScore(torch, dev)
    for _ in range(2):
        ps.launch()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()   # torch's current stream, which is the stream the op launches on
    for _ in range(reps):
        ps.launch()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    gbs = ps.algorithmic_bytes() / (us * 1e-6) / 1e9
    tflops = ps.flops() / (us * 1e-6) / 1e12
    res = {"workload": f"B={ps.B}, KG={ps.KG}, T=L={ps.T} causal, nh={ps.nh}, r={ps.r}, fp16 keys, fp32 scores",
           "avg_launch_us": us, "algorithmic_bytes": ps.algorithmic_bytes(), "gbs": gbs,
           "hbm_frac": gbs / PEAK_HBM_GBS, "tflops": tflops, "mfma_frac_of_peak": tflops / PEAK_MFMA_F16_TFLOPS,
           "mfma_busy_frac": mfma_busy_from_profile(), "bound": "hbm (score writes)"}
    del ps
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------------------------------------------------------------
# microbenchmark sweeps of configs[1] and configs[2]
# ---------------------------------------------------------------------------------------------------------------------
COLD_BYTES = 1 << 30   # rotate over input copies of at least this many bytes, so reads come from HBM, not the caches


def time_rotating(torch, launch, copies, reps=10):
    """launch(i) runs one kernel on copy i; one graph launches every copy once; returns µs per launch."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(copies):
            launch(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(copies):
            launch(i)
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * copies)


def sweep_lightning_topk(torch, dev, emit):
    """batch {1, 8, 32} x L {4K, 16K, 64K, 128K}, 4 index heads of r = 32, fp16 keys ~ N(0, 1/32),
    q ~ N(0, 1), w ~ U(0, 1), ReLU, k = L / 32; 2 % of each row's positions get +3 sigma of that row's scores before
    the top-k. Key groups G_I = 1 (one shared index per sequence) and 8 (one per KV group)."""
    from attention_lab import _native as nat
    from attention_lab import hip_select
    for KG in (1, 8):
        for B in (1, 8, 32):
            for L in (4096, 16384, 65536, 131072):
                nh, k = 4, L // 32
                gen = torch.Generator(device=dev)
                gen.manual_seed(B * L + KG)
                per = B * KG * L * 64
                copies = max(2, min(16, -(-COLD_BYTES // per)))
                keys = [(torch.randn(B, KG, L, 32, device=dev, generator=gen) / 32 ** 0.5).to(torch.float16)
                        for _ in range(copies)]
                q = torch.randn(B, KG, nh, 32, device=dev, generator=gen)
                w = torch.rand(B, KG, nh, device=dev, generator=gen)
                sc = [torch.empty(B * KG, L, device=dev) for _ in range(copies)]
                stream = lambda: torch.cuda.current_stream(dev).cuda_stream

                def score(i):
                    nat.call("attnlab_score_lightning", keys[i].data_ptr(), nat.DT_F16, q.data_ptr(), w.data_ptr(),
                             sc[i].data_ptr(), L, B, KG, L, 32, nh, 0, L, 1, stream())
                us_score = time_rotating(torch, score, copies)
                for i in range(copies):   # heavy tail: +3 sigma on 2 % of each row's positions
                    mask = torch.rand(B * KG, L, device=dev, generator=gen) < 0.02
                    sc[i] += mask * (3.0 * sc[i].std(dim=1, keepdim=True))
                idx = torch.empty(B * KG, k, dtype=torch.int32, device=dev)
                val = torch.empty(B * KG, k, device=dev)
                # the selection hip_select.topk runs for these rows: tiled over the chip for 8K..256K scores (state
                # zeroed once, left zeroed by every call), one workgroup per row below
                state = torch.zeros(B * KG, nat.SELECT_STATE_WORDS, dtype=torch.int32, device=dev)
                nbytes = nat.lib().attnlab_select_scratch_bytes(B * KG, L, k, nat.ORDER_SCORE)
                scratch = torch.empty(max(nbytes, 4), dtype=torch.uint8, device=dev)
                tiled = hip_select.use_tiled(B * KG, L)

                def select(i):
                    if tiled:
                        nat.call("attnlab_topk_tiled", sc[i].data_ptr(), L, B * KG, L, k, nat.ORDER_SCORE,
                                 idx.data_ptr(), val.data_ptr(), k, state.data_ptr(), scratch.data_ptr(), nbytes,
                                 stream())
                    else:
                        nat.call("attnlab_topk", sc[i].data_ptr(), L, B * KG, L, k, nat.ORDER_SCORE, idx.data_ptr(),
                                 val.data_ptr(), k, stream())
                us_topk = time_rotating(torch, select, copies)

                def torch_topk(i):   # the reference's own top-k (decode.py:86-93) on the same rows, for comparison
                    torch.topk(sc[i], k, dim=-1, sorted=True)
                try:   # graph replays time the GPU work; eager launches where torch.topk cannot be captured
                    us_torch, torch_mode = time_rotating(torch, torch_topk, copies), "graph"
                except RuntimeError:
                    torch.cuda.synchronize()
                    torch_topk(0)
                    torch.cuda.synchronize()
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for rep in range(10):
                        for i in range(copies):
                            torch_topk(i)
                    e1.record()
                    torch.cuda.synchronize()
                    us_torch, torch_mode = e0.elapsed_time(e1) * 1e3 / (10 * copies), "eager"
                score_bytes = B * KG * (L * 64 + L * 4) + B * KG * nh * (32 * 4 + 4)
                topk_bytes = B * KG * (4 * L + 8 * k)
                emit({"sweep": "lightning_score_topk", "batch": B, "key_groups": KG, "L": L, "k": k,
                      "topk_kernels": "tiled (histogram, classify, resolve)" if tiled else "one workgroup per row",
                      "score_us": us_score, "score_gbs": score_bytes / us_score / 1e3,
                      "score_frac": score_bytes / us_score / 1e3 / PEAK_HBM_GBS,
                      "topk_us": us_topk, "topk_gbs": topk_bytes / us_topk / 1e3, "torch_topk_us": us_torch,
                      "torch_topk_timing": torch_mode})
                del keys, sc
                torch.cuda.empty_cache()


def sweep_attend(torch, dev, emit):
    """L = 32K, 8 KV groups x 2 query heads, d = 128, bf16 K/V ~ N(0, 1); rows = 4 sinks + the 128 most
    recent positions + k uniform picks from the rest (S = 132 + k), k in {64, 256, 1024, 2048}, batch {1, 16}, rows
    sorted and unsorted; against the dense decode kernel at the same shape."""
    from attention_lab import _native as nat
    from attention_lab import hip_attend
    L, G, h, d = 32768, 8, 2, 128
    for B in (1, 16):
        per = B * G * L * d * 2 * 2
        copies = max(2, min(16, -(-COLD_BYTES // per)))
        gen = torch.Generator(device=dev)
        gen.manual_seed(B)
        K = [torch.randn(B, G, L, d, device=dev, generator=gen, dtype=torch.bfloat16) for _ in range(copies)]
        V = [torch.randn(B, G, L, d, device=dev, generator=gen, dtype=torch.bfloat16) for _ in range(copies)]
        q = torch.randn(B, G, h, d, device=dev, generator=gen, dtype=torch.bfloat16)
        out = torch.empty(B, G, h, d, device=dev, dtype=torch.bfloat16)
        stream = lambda: torch.cuda.current_stream(dev).cuda_stream
        BG = B * G
        Pd = hip_attend.dense_partitions(BG, L)
        part = torch.empty(BG * max(64, Pd) * h * 130, device=dev)

        def dense(i):
            nat.call("attnlab_dense_decode", K[i].data_ptr(), V[i].data_ptr(), L * d, d, q.data_ptr(), B, G, h, L, L,
                     Pd, 1.0 / math.sqrt(d), out.data_ptr(), 1, part.data_ptr(), stream())
        us_dense = time_rotating(torch, dense, copies)
        for k in (64, 256, 1024, 2048):
            S = 132 + k
            P = hip_attend.sparse_partitions(BG, S, h)
            base = torch.cat([torch.arange(4, device=dev), torch.arange(L - 128, L, device=dev)])
            res = {}
            for order in ("sorted", "unsorted"):
                rows = []
                for _ in range(copies):
                    pick = torch.rand(BG, L - 132, device=dev, generator=gen).topk(k, dim=1).indices + 4
                    r = torch.cat([base.expand(BG, 132), pick], dim=1)
                    r = r.sort(dim=1).values if order == "sorted" else r[:, torch.randperm(S, device=dev)]
                    rows.append(r.to(torch.int32).contiguous())

                def att(i):
                    nat.call("attnlab_attend", K[i].data_ptr(), V[i].data_ptr(), L * d, d, q.data_ptr(),
                             rows[i].data_ptr(), S, B, G, h, S, L, P, 1.0 / math.sqrt(d), out.data_ptr(), 1,
                             part.data_ptr(), stream())
                res[order] = time_rotating(torch, att, copies)
            ab = BG * (S * d * 2 * 2 + 4 * S + 2 * h * d * 2)
            emit({"sweep": "attend", "batch": B, "L": L, "k": k, "rows": S, "partitions": P,
                  "sorted_us": res["sorted"], "unsorted_us": res["unsorted"],
                  "sorted_gbs": ab / res["sorted"] / 1e3, "dense_us": us_dense,
                  "speedup_vs_dense": us_dense / max(res["sorted"], res["unsorted"])})
        del K, V
        torch.cuda.empty_cache()


def qwen3_1p7b(torch, dev, seed):
    """BASELINE configs[3]'s model shape with random bf16 weights ~ N(0, 0.02) (transformers' own init), on `dev`."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=151936, hidden_size=2048, intermediate_size=6144, num_hidden_layers=28,
                      num_attention_heads=16, num_key_value_heads=8, head_dim=128, max_position_embeddings=40960,
                      rope_theta=1_000_000.0, rms_norm_eps=1e-6, tie_word_embeddings=True, initializer_range=0.02,
                      attn_implementation="sdpa")
    torch.manual_seed(seed)
    with torch.device(dev):
        model = Qwen3ForCausalLM(cfg)
    model = model.to(torch.bfloat16).eval()
    for p in model.parameters():
        p.requires_grad_(False)
    return model


def qwen3_8b(torch, dev, seed):
    """BASELINE configs[4]'s model shape (36 layers, hidden 4096, 32q/8kv, d=128, FFN 12288, vocab 151936) with random
    bf16 weights ~ N(0, 0.02) (transformers' own init), on `dev`."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=151936, hidden_size=4096, intermediate_size=12288, num_hidden_layers=36,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=128, max_position_embeddings=40960,
                      rope_theta=1_000_000.0, rms_norm_eps=1e-6, tie_word_embeddings=False, initializer_range=0.02,
                      attn_implementation="sdpa")
    torch.manual_seed(seed)
    with torch.device(dev):
        model = Qwen3ForCausalLM(cfg)
    model = model.to(torch.bfloat16).eval()
    for p in model.parameters():
        p.requires_grad_(False)
    torch.cuda.empty_cache()
    return model


def logit_agreement(torch, a, b):
    """a, b: [n, V] float32 logits of the same positions."""
    lp, lq = torch.log_softmax(b, -1), torch.log_softmax(a, -1)
    return {"top1_agreement": float((a.argmax(-1) == b.argmax(-1)).float().mean()),
            "max_abs_diff": float((a - b).abs().max()),
            "rel_norm_diff": float((a - b).norm() / b.norm()),
            "kl_mean": float((lp.exp() * (lp - lq)).sum(-1).mean())}


def run_c5(torch, dev, args):
    """configs[4] through the wrapper on the HIP kernels: one chunked prefill of B x L uniform random ids (index table
    built on the way), greedy decode on the full read (A), rollback, the same tokens (teacher-forced) on the sparse
    read (D0, rho = 1/32), and a few steps with k0 = capacity (every candidate selected, which must equal A). Per-step
    times are eager wall clock (the model's own layers launch from Python), each step ending in a synchronize."""
    from attention_lab.qwen_wrap import LabRunner, LabState, make_state, wrap_model
    B, L, steps, chunk = args.c5_batch, args.c5_context, args.c5_steps, args.c5_chunk
    t_setup = time.perf_counter()
    model = qwen3_8b(torch, dev, args.seed)
    holder = wrap_model(model)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    prompt = torch.randint(0, model.config.vocab_size, (B, L), device=dev, generator=gen)
    cap = L + steps + 1
    print(f"[c5] model ready in {time.perf_counter() - t_setup:.1f}s", file=sys.stderr, flush=True)
    res = {}
    with torch.inference_mode():
        sparse = make_state(model, cap, "sparse", selector="index", r=32, seed=args.seed, batch=B)
        cache = sparse.cache
        res["cache_gb"] = round(cache.bytes()["total_bytes"] / 1e9, 2)
        runner = LabRunner(model, holder, sparse)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        logits = None
        seg = max(chunk, L // 8)
        for a in range(0, L, seg):
            logits = runner.prefill(prompt[:, a:a + seg], chunk)
            torch.cuda.synchronize()
            print(f"[c5] prefill {a + prompt[:, a:a + seg].shape[1]}/{L} ({time.perf_counter() - t0:.1f}s)",
                  file=sys.stderr, flush=True)
        res["prefill_s"] = round(time.perf_counter() - t0, 2)
        res["prefill_tok_s"] = round(B * L / res["prefill_s"], 1)
        first = logits[:, -1].argmax(-1, keepdim=True)

        def decode(run, feed, n):
            """n steps; feed(i, last_logits) -> token ids [B, 1]; returns ([n, B, V] logits, tokens, ms per step)."""
            outs, toks, times = [], [], []
            lg = None
            for i in range(n):
                tok = feed(i, lg)
                toks.append(tok)
                torch.cuda.synchronize()
                t = time.perf_counter()
                lg = run.step(tok)[:, -1].float()
                torch.cuda.synchronize()
                times.append(time.perf_counter() - t)
                outs.append(lg)
            warm = times[2:] if len(times) > 4 else times
            return torch.stack(outs), toks, 1e3 * sum(warm) / len(warm)

        full = LabRunner(model, holder, LabState(cache, sparse.indexers, mode="full"))
        full_logits, tokens, res["decode_ms_full"] = decode(
            full, lambda i, lg: first if i == 0 else lg.argmax(-1, keepdim=True), steps)
        print(f"[c5] full read: {res['decode_ms_full']:.2f} ms per step", file=sys.stderr, flush=True)
        cache.rollback(L)
        res["k0"] = sparse.begin_request(args.rho)
        sp_logits, _, res["decode_ms_sparse"] = decode(runner, lambda i, lg: tokens[i], steps)
        print(f"[c5] sparse read: {res['decode_ms_sparse']:.2f} ms per step", file=sys.stderr, flush=True)
        res["sparse_vs_full"] = logit_agreement(torch, sp_logits.flatten(0, 1), full_logits.flatten(0, 1))
        cache.rollback(L)
        n_all = min(4, steps)
        allk = LabState(cache, sparse.indexers, mode="sparse", selector="index", canonical_order=True)
        allk.begin_request(args.rho, k0=cap)
        all_logits, _, _ = decode(LabRunner(model, holder, allk), lambda i, lg: tokens[i], n_all)
        res["sparse_k0_capacity_vs_full"] = logit_agreement(torch, all_logits.flatten(0, 1),
                                                            full_logits[:n_all].flatten(0, 1))
        cache.rollback(L)

        def graph_step(run, tok, reps=20):
            """The whole-model step at legal length L + 1 captured in one HIP graph and replayed `reps` times (each
            replay rewrites the same cache slot): GPU time per step without the eager launch overhead. Returns (ms,
            replay output == eager output)."""
            run.step(tok)                      # allocations and workspaces before the capture
            cache.rollback(L)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                out = run.step(tok)
            cache.rollback(L)
            g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            got = out.clone()
            want = run.step(tok)
            cache.rollback(L)
            torch.cuda.synchronize()
            del g
            return e0.elapsed_time(e1) / reps, bool(torch.equal(got, want))

        res["graph_ms_full"], res["graph_full_equals_eager"] = graph_step(full, tokens[0])
        res["graph_ms_sparse"], res["graph_sparse_equals_eager"] = graph_step(runner, tokens[0])
        print(f"[c5] graph steps: full {res['graph_ms_full']:.2f} ms, sparse {res['graph_ms_sparse']:.2f} ms",
              file=sys.stderr, flush=True)
    res["graph_tok_s_full"] = round(B * 1e3 / res["graph_ms_full"], 1)
    res["graph_tok_s_sparse"] = round(B * 1e3 / res["graph_ms_sparse"], 1)
    res["graph_sparse_speedup"] = round(res["graph_ms_full"] / res["graph_ms_sparse"], 3)
    res["tok_s_full"] = round(B * 1e3 / res["decode_ms_full"], 1)
    res["tok_s_sparse"] = round(B * 1e3 / res["decode_ms_sparse"], 1)
    res["sparse_speedup"] = round(res["decode_ms_full"] / res["decode_ms_sparse"], 3)
    print(json.dumps({
        "workload": f"configs[4]: random-init Qwen3-8B shape (36 layers, hidden 4096, 32q/8kv, d=128, FFN 12288, "
                    f"vocab 151936, bf16 ~ N(0, 0.02)), batch {B} x {L}-token uniform random context, {steps} greedy "
                    f"steps on the full read, the same tokens on the sparse read (rho={args.rho}, one r=32 grouped "
                    f"indexer per layer) and {n_all} on the sparse read with k0 = capacity; whole model on the GPU, "
                    f"attention through the HIP kernels; decode_ms_* are eager per-step wall clock (the model's layers launch from "
                    f"Python), graph_ms_* one whole step at legal length {L} + 1 replayed from a HIP graph",
        **res,
        "note": "untrained indexers pick rows unrelated to the attention scores, so sparse_vs_full measures the 1/32 "
                "read's departure, not a quality result; k0 = capacity must reproduce the full read up to bf16 "
                "rounding and summation order",
    }))
    return 0


def run_f32_workload(torch, dev, args, layers=8):
    """attnlab_sparse_decode_step_f32 (float32 zT / wq_t / wk / index query and key, bf16 K/V) and the bf16 step on the
    same shape: B x G x L of the bench line, k from rho, position order, graphs of `layers` rotating layers. Reports
    us per layer and the fp32 scan's table bytes (r * 4 per candidate column)."""
    from attention_lab import _native as nat
    from attention_lab import hip_attend
    from attention_lab.indexer import GroupedIndexer
    from attention_lab.selection import fixed_budget, selection_layout
    B, G, h, d, r, L = args.batch, args.groups, args.heads_per_group, 128, args.index_dim, args.context
    lay = selection_layout(L)
    lo, hi, k = lay.candidate_lo, lay.candidate_hi, lay.clamp_k(fixed_budget(L, args.rho))
    S, C, M = lay.fixed_count + k, L, lay.candidate_count
    lib = nat.lib()
    P = hip_attend.sparse_partitions(B * G, S, h, merged=True)
    ws_bytes = lib.attnlab_sparse_decode_workspace(B, G, h, lo, hi, L, k, P)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    state = torch.zeros(B * G * nat.SELECT_STATE_WORDS, dtype=torch.int32, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    K = [torch.randn(B, G, C, d, generator=gen, device=dev).to(torch.bfloat16) for _ in range(layers)]
    V = [torch.randn(B, G, C, d, generator=gen, device=dev).to(torch.bfloat16) for _ in range(layers)]
    q = torch.randn(B, G, h, d, generator=gen, device=dev).to(torch.bfloat16)
    out = torch.empty(B, G, h, d, dtype=torch.bfloat16, device=dev)
    res = {"f32_workload": f"sparse step B={B} G={G} h={h} L={L} r={r} k={k} S={S} P={P}, {layers} rotating layers"}
    for dt, entry in ((torch.float32, "attnlab_sparse_decode_step_f32"), (torch.bfloat16, "attnlab_sparse_decode_step")):
        zT = [torch.randn(B, G, r, C, generator=gen, device=dev).to(dt) for _ in range(layers)]
        idx = GroupedIndexer(G, h, d, r, device=dev, dtype=dt, seed=args.seed)
        q_cat = torch.randn(B, G, h * d, generator=gen, device=dev).to(dt)
        k_new = torch.randn(B, G, d, generator=gen, device=dev).to(dt)

        def step(l):
            nat.call(entry, q.data_ptr(), q_cat.data_ptr(), K[l].data_ptr(), V[l].data_ptr(), zT[l].data_ptr(),
                     idx.wq_t_scaled.data_ptr(), idx.wk.data_ptr(), k_new.data_ptr(), B, G, h, r, C, lo, hi, L, k,
                     L - 1, 1.0 / math.sqrt(d), nat.ORDER_POSITION, P, state.data_ptr(), ws.data_ptr(), ws_bytes,
                     None, None, out.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)

        name = "float32" if dt == torch.float32 else "bfloat16"
        res[f"{name}_us_per_layer"] = round(time_rotating(torch, step, layers, reps=20), 2)
        res[f"{name}_table_bytes_per_layer"] = B * G * r * M * zT[0].element_size()
        del zT
        torch.cuda.empty_cache()
    print(json.dumps(res), flush=True)
    return 0


def p_geometry(N0, rho):
    """Legal length N0 + 1, capacity N0 + 128, the selection layout and k of the reference's P0/P1 benches."""
    from attention_lab.selection import fixed_budget, selection_layout
    L, C = N0 + 1, N0 + 128
    lay = selection_layout(L)
    k = lay.clamp_k(fixed_budget(L, rho))
    return L, C, lay, k


def run_p0(torch, dev, args):
    """bench/p0_score_kernel.py on this build: the D chain's scoring segment (z column of the newest key, u, the scores
    of every candidate) per layer, batch 1. Strategies: pytorch_chain (project_keys + column copy + project_queries +
    candidate_scores, bf16 matmuls on the GPU), pytorch_score_only (candidate_scores from a precomputed u),
    fused_1launch (HipScore.fused) and fused_2launch (HipScore.two_launch). Each is a graph over `layers` index tables
    timed with HIP events. Numerics on layer 0: fused fp32 scores against an fp32 matmul of the same bf16 values, the
    z column against the RNE of its fp32 value, top-k set agreement with the chain's bf16 scores. The stop gate is the
    reference's (p0_score_kernel.py:33)."""
    from attention_lab.hip_score import HipScore
    from attention_lab.indexer import GroupedIndexer
    gate = {"fused_us_max_32k": 80.0, "ratio_vs_chain_max": 0.75, "scores_atol": 1e-5, "scores_rel_norm": 1e-5,
            "z_rel_ulp": 2.0 ** -8}
    hs, bf = HipScore(), torch.bfloat16
    G, h, d, r, nl = 8, 2, 128, 32, args.p_layers
    blocks = []
    for N0 in args.p_lengths:
        L, C, lay, k = p_geometry(N0, args.rho)
        lo, hi, wc, M = lay.candidate_lo, lay.candidate_hi, L - 1, lay.candidate_count
        gen = torch.Generator(device=dev)
        gen.manual_seed(args.seed + N0)
        zT = [torch.randn(G, r, C, generator=gen, device=dev).to(bf) for _ in range(nl)]
        k_new = torch.randn(G, d, generator=gen, device=dev).to(bf)
        q_cat = torch.randn(G, h * d, generator=gen, device=dev).to(bf)
        idx = GroupedIndexer(G, h, d, r, device=dev, dtype=bf, seed=args.seed)
        wk, wq_t = idx.wk, idx.wq_t_scaled
        outs = [torch.empty(G, M, dtype=torch.float32, device=dev) for _ in range(nl)]
        ubufs = [torch.empty(G, r, dtype=torch.float32, device=dev) for _ in range(nl)]
        u_pre = torch.matmul(q_cat.unsqueeze(1), wq_t)                       # [G, 1, r]
        kcol = k_new.unsqueeze(-1).contiguous()                               # [G, d, 1]

        def chain(i):
            zT[i][:, :, wc:wc + 1].copy_(torch.matmul(wk, kcol))
            u = torch.matmul(q_cat.unsqueeze(1), wq_t)
            return torch.matmul(u, zT[i][:, :, lo:hi])

        strategies = {
            "pytorch_chain": chain,
            "pytorch_score_only": lambda i: torch.matmul(u_pre, zT[i][:, :, lo:hi]),
            "fused_1launch": lambda i: hs.fused(zT[i], k_new, wk, q_cat, wq_t, lo, hi, wc, out=outs[i]),
            "fused_2launch": lambda i: hs.two_launch(zT[i], k_new, wk, q_cat, wq_t, lo, hi, wc, out=outs[i],
                                                     u_buf=ubufs[i]),
        }
        us = {name: time_rotating(torch, fn, nl) for name, fn in strategies.items()}
        # numerics on layer 0
        z0 = zT[0].clone()
        fused = hs.fused(z0, k_new, wk, q_cat, wq_t, lo, hi, wc)
        u32 = torch.matmul(q_cat.float().unsqueeze(1), wq_t.float())
        ref = torch.matmul(u32, zT[0].float()[:, :, lo:hi]).squeeze(1)
        diff = (fused - ref).abs()
        atol, rel = float(diff.max()), float(diff.norm() / ref.norm())
        zref = torch.matmul(wk.float(), k_new.float().unsqueeze(-1)).squeeze(-1)
        zgot = z0[:, :, wc].float()
        z_rel = float(((zgot - zref).abs() / zref.abs().clamp_min(1e-30)).max())
        z_bits = float((z0[:, :, wc] == zref.to(bf)).float().mean())
        chain_scores = chain(0).squeeze(1).float()
        kk = max(1, k)
        a_idx = torch.topk(fused, kk, dim=-1).indices
        b_idx = torch.topk(chain_scores, kk, dim=-1).indices
        agree = float(sum(len(set(a.tolist()) & set(b.tolist())) for a, b in zip(a_idx, b_idx)) / (G * kk))
        torch.cuda.synchronize()
        num = {"scores_max_abs": atol, "scores_rel_norm": rel, "z_max_rel": z_rel, "z_bitwise_rne": z_bits,
               "topk_agreement_vs_chain_bf16": agree,
               "pass": atol <= gate["scores_atol"] and rel <= gate["scores_rel_norm"] and z_rel <= gate["z_rel_ulp"]}
        block = {"bench": "p0", "N0": N0, "legal": L, "capacity": C, "candidates": M, "k": k, "layers": nl,
                 "us_per_layer": {n: round(v, 2) for n, v in us.items()}, "numerics": num}
        print(json.dumps(block), flush=True)
        blocks.append(block)
        del zT, outs
        torch.cuda.empty_cache()
    big = [b for b in blocks if b["N0"] >= 32000]
    g = {"gate": gate, "numerics_pass_all": all(b["numerics"]["pass"] for b in blocks)}
    if big:
        b = big[-1]
        fused_us = min(b["us_per_layer"]["fused_1launch"], b["us_per_layer"]["fused_2launch"])
        g.update({"evaluated_at_N0": b["N0"], "fused_us": fused_us,
                  "ratio_vs_chain": round(fused_us / b["us_per_layer"]["pytorch_chain"], 4)})
        g["pass"] = (g["numerics_pass_all"] and fused_us <= gate["fused_us_max_32k"]
                     and g["ratio_vs_chain"] <= gate["ratio_vs_chain_max"])
    print(json.dumps({"bench": "p0", "summary": g}), flush=True)
    return 0


def run_p1(torch, dev, args):
    """bench/p1_attend_kernel.py on this build: the read of the S selected K and V rows and the attention over them,
    batch 1, G=8, h=2. Rows are F and k random distinct candidates per layer and group (cat order), prepared outside
    the timed region. Strategies: pytorch_gather (flat index_select of K and of V, then subset attention as bf16
    matmuls with the transposed K made contiguous, softmax in fp32), fused_attend_P{1,2,4,8} (HipAttend, bf16 output)
    and, as context only, the dense kernel over the legal length. Graphs over `layers` caches, HIP events. Numerics on
    layer 0: the fp32 kernel output against an fp32 masked softmax over the same rows, the bf16 output against the
    RNE of the fp32 output. The stop gate is the reference's (p1_attend_kernel.py:32)."""
    from attention_lab import hip_attend
    gate = {"fused_us_max_at_S1076": 60.0, "ratio_vs_gather_sdpa_max": 0.80, "out_atol": 5e-5, "out_rel_norm": 1e-5,
            "bf16_ulp": 2.0 ** -8}
    ha, bf = hip_attend.HipAttend(), torch.bfloat16
    G, h, d, nl = 8, 2, 128, args.p_layers
    scale = 1.0 / math.sqrt(d)
    blocks = []
    for N0 in args.p_lengths:
        L, C, lay, k = p_geometry(N0, args.rho)
        S = lay.fixed_count + k
        gen = torch.Generator(device=dev)
        gen.manual_seed(args.seed + N0)
        K = [torch.randn(G, C, d, generator=gen, device=dev).to(bf) for _ in range(nl)]
        V = [torch.randn(G, C, d, generator=gen, device=dev).to(bf) for _ in range(nl)]
        q = torch.randn(G, h, d, generator=gen, device=dev).to(bf)
        fixed = torch.tensor(lay.fixed_positions(), device=dev, dtype=torch.long)
        rows, flats = [], []
        for _ in range(nl):
            pick = torch.stack([torch.randperm(lay.candidate_count, generator=gen, device=dev)[:k] for _ in range(G)])
            r32 = torch.cat([fixed.expand(G, -1), pick + lay.candidate_lo], dim=1).to(torch.int32).contiguous()
            rows.append(r32)
            flats.append((r32.long() + torch.arange(G, device=dev).view(G, 1) * C).reshape(-1))
        outb = torch.empty(G, h, d, dtype=bf, device=dev)
        part = torch.empty(G * 8 * h * (d + 2), dtype=torch.float32, device=dev)

        def gather(i):
            ks = K[i].reshape(G * C, d).index_select(0, flats[i]).view(G, S, d)
            vs = V[i].reshape(G * C, d).index_select(0, flats[i]).view(G, S, d)
            sc = torch.matmul(q, ks.transpose(1, 2).contiguous()).float() * scale
            return torch.matmul(torch.softmax(sc, -1).to(bf), vs)

        strategies = {"pytorch_gather": gather}
        for P in (1, 2, 4, 8):
            strategies[f"fused_attend_P{P}"] = (lambda P: lambda i: ha(K[i], V[i], q, rows[i], partitions=P,
                                                                       out_dtype=bf, out=outb, part=part))(P)
        strategies["dense_full_context"] = lambda i: hip_attend.dense_decode(q.unsqueeze(0), K[i].unsqueeze(0),
                                                                             V[i].unsqueeze(0), L)
        us = {name: time_rotating(torch, fn, nl) for name, fn in strategies.items()}
        # numerics on layer 0
        o32 = ha(K[0], V[0], q, rows[0], partitions=4, out_dtype=torch.float32)
        o16 = ha(K[0], V[0], q, rows[0], partitions=4, out_dtype=bf)
        kf, vf = K[0].float(), V[0].float()
        s = torch.matmul(q.float(), kf.transpose(1, 2).contiguous()) * scale        # [G, h, C] fp32
        mask = torch.full((G, 1, C), float("-inf"), device=dev)
        mask.scatter_(2, rows[0].long().unsqueeze(1), 0.0)
        ref = torch.matmul(torch.softmax(s + mask, -1), vf)
        diff = (o32 - ref).abs()
        atol, rel = float(diff.max()), float(diff.norm() / ref.norm())
        bits = float((o16 == o32.to(bf)).float().mean())
        ulp = float(((o16.float() - o32).abs() / o32.abs().clamp_min(1e-30)).max())
        torch.cuda.synchronize()
        num = {"out_max_abs": atol, "out_rel_norm": rel, "bf16_equal_rne": bits, "bf16_max_rel": ulp,
               "pass": atol <= gate["out_atol"] and rel <= gate["out_rel_norm"] and ulp <= gate["bf16_ulp"]}
        block = {"bench": "p1", "N0": N0, "legal": L, "capacity": C, "k": k, "S": S, "layers": nl,
                 "us_per_layer": {n: round(v, 2) for n, v in us.items()}, "numerics": num}
        print(json.dumps(block), flush=True)
        blocks.append(block)
        del K, V
        torch.cuda.empty_cache()
    big = [b for b in blocks if b["N0"] >= 32000]
    g = {"gate": gate, "numerics_pass_all": all(b["numerics"]["pass"] for b in blocks)}
    if big:
        b = big[-1]
        fused = {n: v for n, v in b["us_per_layer"].items() if n.startswith("fused")}
        best = min(fused, key=fused.get)
        g.update({"evaluated_at_S": b["S"], "best": best, "fused_us": fused[best],
                  "ratio_vs_gather": round(fused[best] / b["us_per_layer"]["pytorch_gather"], 4)})
        g["pass"] = (g["numerics_pass_all"] and fused[best] <= gate["fused_us_max_at_S1076"]
                     and g["ratio_vs_gather"] <= gate["ratio_vs_gather_sdpa_max"])
    print(json.dumps({"bench": "p1", "summary": g}), flush=True)
    return 0


def run_c4(torch, dev, args):
    """configs[3] through the wrapper on the HIP kernels: greedy decode on the full read (A); the same tokens on the
    sparse read (D0, rho = 1/32) and on the sparse read with k0 = capacity (every candidate selected, which must
    equal A); the full read against the unwrapped model in float32 with transformers' eager attention."""
    from attention_lab.qwen_wrap import LabRunner, make_state, unwrap_model, wrap_model
    T0, steps = args.c4_prompt, args.c4_steps
    t_setup = time.perf_counter()
    model = qwen3_1p7b(torch, dev, args.seed)
    holder = wrap_model(model)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    prompt = torch.randint(0, model.config.vocab_size, (1, T0), device=dev, generator=gen)
    cap = T0 + steps + 1
    print(f"[c4] model ready in {time.perf_counter() - t_setup:.1f}s", file=sys.stderr, flush=True)

    def timed(fn):
        torch.cuda.synchronize()
        t = time.perf_counter()
        out = fn()
        torch.cuda.synchronize()
        return out, time.perf_counter() - t

    def compare(a, b):
        """a, b: [steps, V] float32 logits."""
        lp, lq = torch.log_softmax(b, -1), torch.log_softmax(a, -1)
        return {"top1_agreement": float((a.argmax(-1) == b.argmax(-1)).float().mean()),
                "max_abs_diff": float((a - b).abs().max()),
                "rel_norm_diff": float((a - b).norm() / b.norm()),
                "kl_mean": float((lp.exp() * (lp - lq)).sum(-1).mean())}

    res = {}
    with torch.inference_mode():
        full = LabRunner(model, holder, make_state(model, cap, "full"))
        logits, res["prefill_s_full"] = timed(lambda: full.prefill(prompt, 1024))
        tokens, full_logits = [], []
        tok = logits[:, -1].argmax(-1, keepdim=True)

        def decode_full():
            nonlocal tok
            for _ in range(steps):
                tokens.append(tok)
                lg = full.step(tok)[:, -1].float()
                full_logits.append(lg)
                tok = lg.argmax(-1, keepdim=True)
        _, t = timed(decode_full)
        res["decode_ms_full"] = t * 1e3 / steps
        full_logits = torch.cat(full_logits)
        del full
        print(f"[c4] full read done ({res['prefill_s_full']:.1f}s prefill)", file=sys.stderr, flush=True)

        def sparse_run(k0):
            # k0 = capacity selects up to 8252 candidates: position order (canonical_order) keeps any k
            st = make_state(model, cap, "sparse", selector="index", r=32, seed=args.seed, canonical_order=k0 is not None)
            runner = LabRunner(model, holder, st)
            _, t_pf = timed(lambda: runner.prefill(prompt, 1024))
            k = st.begin_request(args.rho, k0=k0)
            outs = []
            _, t_dec = timed(lambda: [outs.append(runner.step(tokens[i])[:, -1].float()) for i in range(steps)])
            return torch.cat(outs), t_pf, t_dec * 1e3 / steps, k

        sp, res["prefill_s_sparse"], res["decode_ms_sparse"], k0 = sparse_run(None)
        res["sparse_vs_full"] = compare(sp, full_logits)
        allk, _, _, kcap = sparse_run(cap)
        res["sparse_k0_capacity_vs_full"] = compare(allk, full_logits)
        print(f"[c4] sparse reads done (k0 = {k0}, then {kcap})", file=sys.stderr, flush=True)
        del sp, allk
        # reference: the unwrapped model in float32, eager attention, one forward over prompt + generated tokens
        unwrap_model(model)
        ref_model = model.float()
        ref_model.config._attn_implementation = "eager"
        ids = torch.cat([prompt] + tokens, dim=1)
        # logits of positions T0 - 1 .. T0 + steps - 1; step i fed token i at position T0 + i
        ref = ref_model(input_ids=ids, use_cache=False, logits_to_keep=steps + 1).logits[0, 1:].float()
        res["full_vs_float32_eager_reference"] = compare(full_logits, ref)
    print(json.dumps({
        "workload": f"configs[3]: random-init Qwen3-1.7B shape (28 layers, hidden 2048, 16q/8kv, d=128, FFN 6144, "
                    f"vocab 151936, bf16 ~ N(0, 0.02)), {T0}-token uniform prompt, {steps} greedy steps on the full "
                    f"read; the same tokens (teacher-forced) on the sparse read (rho={args.rho}, k0={k0}, one r=32 "
                    f"grouped indexer per layer) and on the sparse read with k0 = capacity; whole model on the GPU, "
                    f"attention through the HIP kernels",
        **res,
        "note": "the indexers are untrained (random), so the rows they pick are unrelated to the attention scores, and "
                "random weights spread the attention mass over the whole context: a 1/32 read then does not reproduce "
                "the full read's logits (sparse_vs_full measures that). k0 = capacity selects every candidate and must "
                "reproduce the full read up to bf16 rounding and summation order",
    }))
    return 0


def run_sweeps(torch, dev, which="all"):
    def emit(d):
        print(json.dumps(d), flush=True)
    if which in ("all", "attend"):
        sweep_attend(torch, dev, emit)
    if which in ("all", "score"):
        sweep_lightning_topk(torch, dev, emit)
    return 0


# ---------------------------------------------------------------------------------------------------------------------
# CPU baseline: the reference's op sequence on the host cores
# ---------------------------------------------------------------------------------------------------------------------
def cpu_info():
    """The host's CPU model and the CPUs this process may use (affinity, capped by a cgroup CPU quota when one is set):
    the all-cores leg runs that many threads, whatever os.cpu_count() reports for the whole machine."""
    model, cores = None, set()
    try:
        phys = None
        with open("/proc/cpuinfo", encoding="utf-8") as f:
            for line in f:
                key, _, val = line.partition(":")
                key, val = key.strip(), val.strip()
                if key == "model name" and model is None:
                    model = val
                elif key == "physical id":
                    phys = val
                elif key == "core id":
                    cores.add((phys, val))
    except OSError:
        pass
    logical = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = logical
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max", encoding="utf-8") as f:
            q, period = f.read().split()[:2]
        if q != "max":
            quota = int(q) / int(period)
    except (OSError, ValueError):
        pass
    usable = affinity if quota is None else max(1, min(affinity, int(quota)))
    return {"cpu_model": model, "logical_cpus": logical, "physical_cores": len(cores) or None,
            "affinity_cpus": affinity, "cgroup_cpu_quota": quota, "usable_cpus": usable}


def _cpu_time(fn, budget_s, min_n=2):
    """Seconds per call of fn over about budget_s seconds (at least min_n calls, after one untimed call)."""
    fn()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or n < min_n:
        fn()
        n += 1
    return (time.perf_counter() - t0) / n, n


def _c1_inputs(torch, seed=0, B=1, G=8, h=2, L=2048, r=32, d=128):
    """configs[0] on the CPU: one Qwen3-0.6B-shaped layer, L=2048, 16q/8kv, bf16 K/V ~ N(0,1), grouped r=32 indexer."""
    from attention_lab.indexer import GroupedIndexer
    g = torch.Generator().manual_seed(seed)
    t = lambda *sh: torch.randn(*sh, generator=g).to(torch.bfloat16)  # noqa: E731
    idx = GroupedIndexer(G, h, d, r, dtype=torch.bfloat16, seed=seed)
    return dict(q=t(B, G, h, 1, d), q_pre=t(B, G, h, 1, d), K=t(B, G, L, d), V=t(B, G, L, d), zT=t(B, G, r, L),
                wq_t=idx.wq_t_scaled, wk=idx.wk, k_new=t(B, G, 1, d), L=L, k0=64)


def _lightning_cpu(torch, keys, q, w, k):
    """configs[1]'s indexer score + top-k on the CPU: s = sum_i w_i ReLU(q_i . key_t), then torch.topk (float32)."""
    s = torch.einsum("gir,gtr->git", q, keys).clamp_min_(0.0)
    s = torch.einsum("gi,git->gt", w, s)
    return torch.topk(s, k, dim=-1)


def cpu_baseline(torch, ls, budget_s, layers_in_step):
    """The reference's op sequence (oracle/ref_path.py: bf16 matmul score, torch.topk, cat, index_select, SDPA) on the
    host cores: layer 0 of the bench shape at all usable CPUs (the headline `value`) and at 1 thread, plus BASELINE's
    B=1 legs: configs[0] (sparse and dense step at L=2048) and configs[1] (lightning score + top-k, L = 4K..32K)."""
    from oracle import ref_path
    info = cpu_info()
    threads_all = info["usable_cpus"]
    prev_threads = torch.get_num_threads()
    B, G, h, d = ls.B, ls.G, ls.h, ls.d
    K, V, zT = ls.K[0].cpu(), ls.V[0].cpu(), ls.zT[0].cpu()
    q = ls.q[0].cpu().view(B, G, h, 1, d)
    q_pre = ls.q_cat[0].cpu().view(B, G, h, 1, d)
    k_new = ls.k_new[0].cpu().view(B, G, 1, d)
    wq_t, wk = ls.wq_t[0].cpu(), ls.wk[0].cpu()
    c1 = _c1_inputs(torch)
    gen = torch.Generator().manual_seed(1)
    c2_cases = []
    for L in (4096, 16384, 32768):
        keys = (torch.randn(8, L, 32, generator=gen) / math.sqrt(32)).to(torch.float16).float()
        c2_cases.append((L, keys, torch.randn(8, 4, 32, generator=gen), torch.rand(8, 4, generator=gen)))
    res = {"kind": "port", "unit": "tok/s", **info}
    out_cpu = rows_cpu = None
    try:
        with torch.inference_mode():
            for threads, tag, share in ((threads_all, "all", 0.45), (1, "one_thread", 0.35)):
                torch.set_num_threads(threads)
                leg = {"threads": threads}

                def step():
                    nonlocal out_cpu, rows_cpu
                    out_cpu, rows_cpu = ref_path.sparse_layer_step(q, q_pre, K, V, zT, wq_t, wk, k_new, ls.L, ls.k0)
                t_layer, n = _cpu_time(step, budget_s * share * 0.8, min_n=1)
                leg.update({"us_per_layer": t_layer * 1e6, "layer_steps": n,
                            "tok_s": ls.B / (layers_in_step * t_layer)})
                if threads == threads_all:
                    t_dense, nd = _cpu_time(lambda: ref_path.dense_layer_step(q, K, V, ls.L), budget_s * 0.1, min_n=1)
                    leg.update({"dense_us_per_layer": t_dense * 1e6, "dense_layer_steps": nd})
                c1_sparse = _cpu_time(lambda: ref_path.sparse_layer_step(c1["q"], c1["q_pre"], c1["K"], c1["V"],
                                                                         c1["zT"], c1["wq_t"], c1["wk"], c1["k_new"],
                                                                         c1["L"], c1["k0"]), budget_s * 0.03)[0]
                c1_dense = _cpu_time(lambda: ref_path.dense_layer_step(c1["q"], c1["K"], c1["V"], c1["L"]),
                                     budget_s * 0.03)[0]
                leg["configs0_b1_l2048_us_per_layer"] = {"sparse": c1_sparse * 1e6, "dense": c1_dense * 1e6}
                leg["configs1_b1_lightning_us"] = {
                    str(L): _cpu_time(lambda: _lightning_cpu(torch, keys, qq, ww, L // 32), budget_s * 0.03)[0] * 1e6
                    for L, keys, qq, ww in c2_cases}
                res[tag] = leg
    finally:
        torch.set_num_threads(prev_threads)
    res.update({"value": res["all"]["tok_s"], "cores": threads_all,
                "sample": (f"{res['all']['layer_steps']} layer-steps of layer 0 (B={ls.B}, L={ls.L}, G={ls.G}, "
                           f"h={ls.h}, k={ls.k}) through the reference's op sequence in bf16 (matmul, torch.topk, "
                           f"cat, index_select, SDPA) on {threads_all} threads, scaled to {layers_in_step} layers; "
                           f"the same at 1 thread in one_thread; B=1 legs of configs[0] and configs[1] in both")})
    return res, out_cpu, rows_cpu


def numerics_vs_cpu(torch, ls, out_cpu, rows_cpu):
    """Layer 0 against the reference's CPU path on the same inputs. The attend is held to the bf16 bar on the CPU
    path's own row lists (identical rows: the GPU gather-free attend over rows_cpu against the CPU's index_select +
    SDPA); the selections are compared separately (the CPU path ranks bf16-rounded scores, the kernel fp32 ones)."""
    from attention_lab import hip_attend
    B, G, h, d = ls.B, ls.G, ls.h, ls.d
    off = (torch.arange(B * G) * ls.C).view(B, G, 1)
    cpu_pos = rows_cpu.view(B, G, -1) - off
    pos = cpu_pos.to(torch.int32).contiguous().to(ls.K[0].device)
    same_rows = hip_attend.attend(ls.q[0], ls.K[0], ls.V[0], pos, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    cpu_out = out_cpu.float().view(B, G, h, d)
    diff = (same_rows.float().cpu() - cpu_out).abs()
    own = (ls.out[0].float().cpu().view(B, G, h, d) - cpu_out).abs()
    gpu_pos = ls.rows.cpu().long()
    agree = [len(set(cpu_pos[b, g].tolist()) & set(gpu_pos[b, g].tolist())) / cpu_pos.shape[-1]
             for b in range(B) for g in range(G)]
    return {"attend_same_rows": {"max_abs": float(diff.max()), "mean_abs": float(diff.mean()),
                                 "bar": {"max_abs": 2e-2, "mean_abs": 2e-3},
                                 "pass": bool(float(diff.max()) <= 2e-2 and float(diff.mean()) <= 2e-3)},
            "row_set_agreement_mean": sum(agree) / len(agree), "row_set_agreement_min": min(agree),
            "own_selection_out": {"max_abs": float(own.max()), "mean_abs": float(own.mean())},
            "note": "attend_same_rows is the bf16 bar on identical row lists; the row-set agreement and "
                    "own_selection_out include the selection difference (bf16-rounded scores on the CPU path, fp32 "
                    "on the GPU) and are not held to that bar"}


# ---------------------------------------------------------------------------------------------------------------------
def run_b1(torch, dev, args):
    """Batch-1 per-layer figures at the reference's headline shape (G=8, h=2) and at h=4, 28 layers rotating, each in
    forward and reverse layer order (median, p95, conservative = the slower order's median)."""
    res = {}
    for hpg in (2, 4):
        ls = LayerStack(torch, dev, batch=1, groups=8, hpg=hpg, context=args.context, layers=28, r=args.index_dim,
                        rho=args.rho, seed=args.seed + 7)
        fns = launchers(ls, torch)
        reps = max(20, args.steps // 2)
        sp = ordered_stats(torch, fns["sparse"], ls.n, reps, 5, per=ls.n)
        dn = ordered_stats(torch, fns["dense"], ls.n, reps, 5, per=ls.n)
        per = kernel_breakdown(torch, fns, ls, args.kernel_reps)
        sparse_bytes = ls.score_bytes() + ls.select_bytes() + ls.attend_bytes()
        us = sp["conservative_us"]
        res[f"h{hpg}"] = {"sparse_us_per_layer": us, "dense_us_per_layer": dn["conservative_us"],
                          "sparse_orders": sp, "dense_orders": dn,
                          "kernel_us": {k: per[k] for k in ("score", "select_attend", "select", "attend",
                                                            "attend_standalone")},
                          "sparse_algorithmic_bytes_per_layer": sparse_bytes,
                          "sparse_gbs": sparse_bytes / (us * 1e-6) / 1e9,
                          "sparse_frac_of_peak": sparse_bytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS}
        del ls, fns
        torch.cuda.empty_cache()
    return res


def attend_head_groups(BG, h, P):
    """The attend's head-group count for BG rows, h heads and P partitions (attend.hip head_groups)."""
    Q = 1
    while h % (2 * Q) == 0 and BG * Q * P < 256:
        Q *= 2
    return Q


def gather_ceiling(torch, dev, args):
    """The attend against the gather-only probe (attnlab_gather_probe: the same rows, grid, lanes and load pipeline,
    no arithmetic) over the row lists the fused step itself selects, one list per layer of the stack, so every layer
    reads other rows of another cache (nothing is served from the Infinity Cache across layers). Both in graphs of one
    launch per layer, both layer orders, conservative medians per layer. The probe also runs at other splits of the same
    rows: Q = 1 with P = 2 (each row loaded once, split over two workgroups) against the attend's Q = 2, P = 1 (each
    row loaded by two head-group workgroups, the second read from L2)."""
    from attention_lab import _native as nat
    from attention_lab import hip_attend
    out = {"probe": "attnlab_gather_probe: the attend's rows, grid, lane layout and 4-stage load pipeline; XOR-fold "
                    "of the loaded words, one word stored per thread"}
    for B, h in ((16, 4), (1, 2)):
        ls = LayerStack(torch, dev, batch=B, groups=args.groups, hpg=h, context=args.context, layers=args.layers,
                        r=args.index_dim, rho=args.rho, seed=args.seed)
        G, d, C, S = ls.G, ls.d, ls.C, ls.S
        lib = nat.lib()
        P = hip_attend.sparse_partitions(B * G, S, h)
        Q = attend_head_groups(B * G, h, P)
        rows = [torch.empty(B * G, S, dtype=torch.int32, device=dev) for _ in range(ls.n)]
        state = torch.zeros(B * G * nat.SELECT_STATE_WORDS, dtype=torch.int32, device=dev)
        wsb = lib.attnlab_sparse_decode_workspace(B, G, h, ls.lo, ls.hi, ls.L, ls.k, P)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        part = torch.empty(B * G * max(P, 2) * h * 130, dtype=torch.float32, device=dev)
        sink = torch.empty(B * G * 8 * 8 * 256, dtype=torch.int32, device=dev)
        scale = 1.0 / math.sqrt(d)

        def stream():
            return torch.cuda.current_stream(dev).cuda_stream

        for l in range(ls.n):   # the step's own selection of every layer, in position order
            nat.call("attnlab_sparse_decode_step", ls.q[l].data_ptr(), ls.q_cat[l].data_ptr(), ls.K[l].data_ptr(),
                     ls.V[l].data_ptr(), ls.zT[l].data_ptr(), ls.wq_t[l].data_ptr(), ls.wk[l].data_ptr(),
                     ls.k_new[l].data_ptr(), B, G, h, ls.r, C, ls.lo, ls.hi, ls.L, ls.k, ls.write_col, scale,
                     nat.ORDER_POSITION, P, state.data_ptr(), ws.data_ptr(), wsb, rows[l].data_ptr(), None,
                     ls.out[l].data_ptr(), stream())
        torch.cuda.synchronize()

        def attend(l):
            nat.call("attnlab_attend", ls.K[l].data_ptr(), ls.V[l].data_ptr(), C * d, d, ls.q[l].data_ptr(),
                     rows[l].data_ptr(), S, B, G, h, S, C, P, scale, ls.out[l].data_ptr(), 1, part.data_ptr(),
                     stream())

        def probe(q, p):
            def fn(l):
                nat.call("attnlab_gather_probe", ls.K[l].data_ptr(), ls.V[l].data_ptr(), C * d, d, rows[l].data_ptr(),
                         S, B, G, S, C, q, p, sink.data_ptr(), stream())
            return fn

        unique = B * G * S * d * 2 * 2   # every listed K and V row once
        res = {"attend": ordered_stats(torch, attend, ls.n, args.kernel_reps, 3, per=ls.n)["conservative_us"]}
        splits = [(Q, P), (1, P * Q)] if Q > 1 else [(Q, P)]
        for q, p in splits:
            res[f"probe_Q{q}_P{p}"] = ordered_stats(torch, probe(q, p), ls.n, args.kernel_reps, 3,
                                                    per=ls.n)["conservative_us"]
        out[f"B{B}_h{h}"] = {"attend_Q_P": [Q, P], "rows_per_bg": S, "unique_row_bytes": unique,
                             "us_per_layer": {k: round(v, 3) for k, v in res.items()},
                             "unique_gbs": {k: round(unique / (v * 1e-6) / 1e9, 1) for k, v in res.items()}}
        print(f"[gather] B={B} h={h}: {out[f'B{B}_h{h}']}", file=sys.stderr, flush=True)
        del ls, rows, ws, part
        torch.cuda.empty_cache()
    print(json.dumps(out))
    return 0


def scan_ceiling(torch, dev, args):
    """The fused score kernel (the step's launch: u, z column, scan, histogram and key lists) against its read probe
    (attnlab_scan_probe: the same grid, u prologue, table loads and load pipeline, with the multiply, reduction,
    histogram and lists replaced by an XOR fold of the loaded words) over the same 36 layers' index tables, in graphs of
    one launch per layer, both layer orders, conservative medians per layer."""
    from attention_lab import _native as nat
    out = {"probe": "attnlab_scan_probe: score_scan_fused's grid, u prologue, table loads and pipeline; XOR-fold of "
                    "the loaded words, one word stored per thread"}
    for B, h in ((16, 4), (1, 2)):
        ls = LayerStack(torch, dev, batch=B, groups=args.groups, hpg=h, context=args.context, layers=args.layers,
                        r=args.index_dim, rho=args.rho, seed=args.seed)
        fns = launchers(ls, torch)
        G, C = ls.G, ls.C
        sink = torch.empty(B * G * ((ls.hi - ls.lo + 16 + 511) // 512) * 256, dtype=torch.int32, device=dev)

        def probe(l):
            nat.call("attnlab_scan_probe", ls.zT[l].data_ptr(), ls.q_cat[l].data_ptr(), ls.wq_t[l].data_ptr(), B, G, C,
                     h * ls.d, ls.lo, ls.hi, sink.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)

        table = B * G * ls.r * (ls.hi - ls.lo) * 2   # every candidate column of every index row, once
        res = {"score": ordered_stats(torch, fns["score"], ls.n, args.kernel_reps, 3, per=ls.n)["conservative_us"],
               "probe": ordered_stats(torch, probe, ls.n, args.kernel_reps, 3, per=ls.n)["conservative_us"]}
        out[f"B{B}_h{h}"] = {"table_bytes": table, "us_per_layer": {k: round(v, 3) for k, v in res.items()},
                             "table_gbs": {k: round(table / (v * 1e-6) / 1e9, 1) for k, v in res.items()},
                             "score_over_probe": round(res["score"] / res["probe"], 4)}
        print(f"[scan] B={B} h={h}: {out[f'B{B}_h{h}']}", file=sys.stderr, flush=True)
        del ls, fns, sink
        torch.cuda.empty_cache()
    print(json.dumps(out))
    return 0


def main() -> int:
    args = parse_args()
    if args.pmc_summary:
        return pmc_summary(*args.pmc_summary)
    if args.pmc_table:
        return pmc_table(args.pmc_table)
    if args.prefill_pmc_summary:
        return prefill_pmc_summary(args.prefill_pmc_summary)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: every GPU box here has one GPU; splitting "
                                   "the step over GPUs (tensor parallel by KV group) is designed, not built or run",
                          "n_gpus": args.gpus}))
        return 2
    import torch
    from attention_lab import _native
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP device"}))
        return 1
    _native.lib()
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False
    if args.pmc_workload:
        return pmc_workload(torch, dev, args)
    if args.prefill_workload:
        return prefill_workload(torch, dev)
    if args.index_build_workload:
        return index_build_workload(torch, dev)
    if args.prefill_attend_workload:
        return prefill_attend_workload(torch, dev)
    if args.sweeps:
        return run_sweeps(torch, dev, args.sweeps)
    if args.c4:
        return run_c4(torch, dev, args)
    if args.c5:
        return run_c5(torch, dev, args)
    if args.gather_ceiling:
        return gather_ceiling(torch, dev, args)
    if args.scan_ceiling:
        return scan_ceiling(torch, dev, args)
    if args.f32_workload:
        return run_f32_workload(torch, dev, args)
    if args.p0:
        return run_p0(torch, dev, args)
    if args.p1:
        return run_p1(torch, dev, args)

    t_setup = time.perf_counter()
    ls = LayerStack(torch, dev, batch=args.batch, groups=args.groups, hpg=args.heads_per_group, context=args.context,
                    layers=args.layers, r=args.index_dim, rho=args.rho, seed=args.seed)
    fns = launchers(ls, torch)
    g_sparse = capture(torch, fns["sparse"], ls.n)
    g_dense = capture(torch, fns["dense"], ls.n)
    print(f"[bench] setup {time.perf_counter() - t_setup:.1f}s: {ls.n} layers, B={ls.B}, L={ls.L}, k={ls.k}, "
          f"S={ls.S}, P={fns['partitions']}, dense P={fns['dense_partitions']}", file=sys.stderr, flush=True)

    # ---- the timed region: exactly `steps` sparse decode steps (an event after every step, no sync between) ----
    for _ in range(args.warmup):
        g_sparse.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    ev[0].record()
    for i in range(args.steps):
        g_sparse.replay()
        ev[i + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_ms = [ev[i].elapsed_time(ev[i + 1]) for i in range(args.steps)]
    ms_step = ev[0].elapsed_time(ev[args.steps]) / args.steps
    value = ls.B * args.steps / (ms_step * args.steps / 1e3)
    print(f"[bench] sparse step {ms_step:.3f} ms ({wall:.2f}s wall for {args.steps} steps)", file=sys.stderr, flush=True)
    # the same steps with the layers in reverse order (the reference's conservative protocol), outside the timed region
    g_rev = capture(torch, fns["sparse"], ls.n, reverse=True)
    rev = replay_stats(torch, g_rev, args.steps, args.warmup)
    del g_rev
    srt = sorted(step_ms)
    timing = {"forward": {"mean_ms": ms_step, "median_ms": statistics.median(step_ms),
                          "p95_ms": srt[min(len(srt) - 1, int(math.ceil(0.95 * len(srt))) - 1)]},
              "reverse": {k: rev[k] for k in ("mean_ms", "median_ms", "p95_ms")},
              "protocol": "HIP events after every graph replay of the 36-layer step; forward = the timed region above, "
                          "reverse = the layers captured in reverse order; conservative = the slower order's median"}
    timing["conservative_ms_per_step"] = max(timing["forward"]["median_ms"], timing["reverse"]["median_ms"])

    dn = ordered_stats(torch, fns["dense"], ls.n, max(10, args.steps // 4), 3)
    ms_dense = dn["conservative_us"] / 1e3
    kus = kernel_breakdown(torch, fns, ls, args.kernel_reps)
    print(f"[bench] dense step {ms_dense:.3f} ms; per-kernel us (conservative medians) "
          f"{({k: round(kus[k], 2) for k in ('score', 'select', 'attend')})}", file=sys.stderr, flush=True)

    sb, selb, ab, db = ls.score_bytes(), ls.select_bytes(), ls.attend_bytes(), ls.dense_bytes()
    score_us = kus["mean"]["score"]   # forward-order mean launch time: what a kernel trace's average measures
    ach = sb / (score_us * 1e-6) / 1e9
    us_layer = ms_step * 1e3 / ls.n
    us_layer_cons = timing["conservative_ms_per_step"] * 1e3 / ls.n
    sparse_bytes = sb + selb + ab
    line = {
        "metric": metric_name(),
        "value": value,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "value_scope": "attention-path tok/s: the sparse read of all 36 layers per step (z append, score, top-k, "
                       "gather-free attend) for B sequences, as one HIP graph; the model's projections, MLP, norms "
                       "and head are not in it, so it is not a whole-model decode rate",
        "config": {"workload": "sparse decode attention read (z append + score + top-k + gather-free attend) over a "
                               "36-layer Qwen3-8B-shaped KV cache, one HIP graph per step; attention-path tok/s",
                   "batch": ls.B, "context": ls.L, "layers": ls.n, "kv_groups": ls.G, "heads_per_group": ls.h,
                   "head_dim": ls.d, "index_dim": ls.r, "rho": args.rho, "k": ls.k, "selected_rows": ls.S,
                   "global_batch": ls.B, "seq_len": ls.L, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "kernel": f"{SCAN_KERNEL} (candidate scan of the index table)", "achieved": ach,
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": ach / PEAK_HBM_GBS,
                     "traffic": measured_traffic() if (ls.B, ls.L, ls.G, ls.r) == (16, 32768, 8, 32) else None,
                     "algorithmic_bytes_per_launch": sb, "avg_launch_us": score_us},
        "timing": timing,
        "per_layer_us": {"sparse": us_layer, "sparse_conservative": us_layer_cons, "dense": ms_dense * 1e3 / ls.n,
                         "score": kus["score"], "select_attend": kus["select_attend"], "select": kus["select"],
                         "attend": kus["attend"], "attend_standalone": kus["attend_standalone"],
                         "select_kernels": fns["select_kernels"],
                         "note": "sparse: the timed region's mean; the kernel figures and dense: conservative medians "
                                 "(slower of forward / reverse layer order); kernel_orders holds every order's median, "
                                 "p95 and mean"},
        "kernel_orders": kus["orders"],
        "hot_path_hbm": {"algorithmic_bytes_per_layer": sparse_bytes, "gbs": sparse_bytes / (us_layer * 1e-6) / 1e9,
                         "frac_of_peak": sparse_bytes / (us_layer * 1e-6) / 1e9 / PEAK_HBM_GBS,
                         "frac_of_peak_conservative": sparse_bytes / (us_layer_cons * 1e-6) / 1e9 / PEAK_HBM_GBS},
        "kernels": {
            "select_attend": {"bytes": selb + ab, "gbs": (selb + ab) / (kus["select_attend"] * 1e-6) / 1e9},
            "select": {"bytes": selb, "gbs": selb / (kus["select"] * 1e-6) / 1e9},
            "attend_standalone": {"bytes": ab, "gbs": ab / (kus["attend_standalone"] * 1e-6) / 1e9},
            "dense": {"bytes": db, "gbs": db / (ms_dense * 1e-3 / ls.n) / 1e9,
                      "frac": db / (ms_dense * 1e-3 / ls.n) / 1e9 / PEAK_HBM_GBS},
        },
        "dense_control": {"tok_s": ls.B / (ms_dense / 1e3), "ms_per_step": ms_dense,
                          "sparse_speedup": ms_dense / ms_step},
    }

    if not args.no_b1:
        try:
            del g_dense
            line["batch1"] = run_b1(torch, dev, args)
        except Exception as e:  # the headline line must still print
            line["batch1"] = {"error": repr(e)}
    if not args.no_prefill:
        try:
            line["prefill_score"] = run_prefill_score(torch, dev)
        except Exception as e:  # the headline line must still print
            line["prefill_score"] = {"error": repr(e)}

    if not args.no_cpu_baseline:
        # layer 0 through the fused step once more so ls.rows holds its row list for the numerics comparison
        fns["score"](0)
        fns["select"](0)
        fns["attend"](0)
        torch.cuda.synchronize()
        cb, out_cpu, rows_cpu = cpu_baseline(torch, ls, args.cpu_seconds, ls.n)
        line["cpu_baseline"] = cb
        line["numerics_vs_cpu_reference_path"] = numerics_vs_cpu(torch, ls, out_cpu, rows_cpu)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
