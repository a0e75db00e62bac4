"""CPU oracle of the sparse-decode hot path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only as the checker
(or, in bench.py, as the timed CPU baseline). The product (attention-lab_amd/) never imports it and has no CPU path.

Modules (each function cites the reference file:line it restates; paths relative to wlvh/attention-lab):
  rules     selection rules (selection.py:21-86)
  bf16      bfloat16 round-to-nearest-even and unpacking in numpy
  exact     float64 restatements: grouped score (indexer.py:15-29, metal_score.py:344-350), z column (RNE,
            metal_score.py:31-40, 84-89), top-k with lowest-index ties (decode.py:86-93 made deterministic), row list
            (decode.py:50-56, 86-93, 160-161), subset attention (metal_attend.py:262-273, reference.py:80-97), dense
            attention (reference.py:51-62, full.py:17-34), causal attention of a prefill chunk (reference.py:28-62,
            legality mask), lightning score and its T-query prefill form with a causal bound (north_star formula,
            no reference code)
  ref_path  the reference's torch op sequence on the CPU (matmul -> topk -> cat -> index_select -> SDPA), the timed
            CPU baseline
  weights   GroupedIndexer's seeded weights (indexer.py:38-45)

How each function is pinned (no function here is "parity unpinned"):
  rules      the known answers of the reference's tests (test_attention_contracts.py:309-347, 237-239, 262;
             test_qwen_wrapper.py:387-392) - tests/test_oracle_pins.py
  exact      closed forms that a dropped term / wrong index / transposed operand breaks (unit-vector queries pick one
             table row, unit rows of wk make project_keys pick one key coordinate per index dim and its columns equal
             z_column of each key, S=1 attention returns the V row, equal scores return the V mean, softmax invariance to a
             shift, k0 = capacity sparse == dense, score == the explicit double loop on tiny inputs), brute force
             (top-k against a full sort, including planted ties, NaN and -0.0), and cross-checks of the two
             independent formulations (masked dense vs listed subset; the masked prefill read vs one sliced dense
             read per query; the batched lightning score vs one single-query score per query, its causal bound
             element by element) - tests/test_oracle_pins.py
  ref_path   agreement with `exact` on the same inputs (set equality for top-k on tie-free scores) -
             tests/test_oracle_pins.py
  weights    golden fixture written by tests/golden/make_golden.py from the reference's own GroupedIndexer -
             tests/test_golden.py
"""
