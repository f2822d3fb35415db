"""CPU oracle of the TriAttention compression path -- TEST INFRASTRUCTURE ONLY.

Nothing in the product imports this package.  It is used by tests/, by
__graft_entry__.smoke() to verify its result, and by bench.py's cpu_baseline leg as
the timed CPU baseline ("port" kind).

Modules
  triattention_ref  torch-CPU restatement of the reference's own torch path
                    (tri/scoring.py, tri/method.py fallback branch,
                    tri/selection.py, tri/cache.py), same ops in the same order.
  brute             float64 brute force (plain loops / numpy) used to pin the
                    restatement on small inputs, and the deterministic
                    (score desc, index asc) selection rule.
  calibration_ref   torch-CPU restatement of the calibration generator's query
                    statistics (_LayerAccumulator.add, pkg/calibration.py:98-131,
                    and the per-layer means of :351-371) with a float64 loop
                    brute force of the definitions.

Parity pins (how each oracle function is checked, see tests/test_oracle_*.py):
  build_geometric_offsets   closed form 2^k <= max
  score_post_rope_keys      reference KATs (tests/test_scoring.py:53-133: slow
                            per-offset reference, scale 4.0, partial-RoPE
                            [2,-5]); float64 brute force; omega=0 closed form
  normalize_head_scores     single-layer closed forms (population variance,
                            1e-6 clamp, head maximum); float64 brute force
  aggregate_layers          tests/test_oracle_aggregate.py: the two-layer
                            closed form of tests/test_selection.py:230-280
                            (mean and max, no collective) from exact power
                            sums; six layers (division by the scoring-layer
                            count); layer 0 counted once; maximum over every
                            KV and query head; nan_to_num mapping after the
                            layer combination (tri/method.py:463-467), NaN-
                            propagating maximum, +inf -> 1e30, -inf kept
  select_keep_indices       reference KATs ([0,1,4,5], v3 evicts {2,5,8,11},
                            uneven quota count); brute-force sort; batched-v3
                            equivalence (tests/test_selection.py:94-125)
  token_slots/materialize   reference KATs ([8,11,0,3], overlapping write,
                            padded page stride: tests/test_cache.py:15-94)
  block-table rewrite       scheduler commit semantics (pkg/stateful.py:327-338)
  shift_positions           reference KATs ([300,20,301] with offsets [172,0] ->
                            [128,20,129]: tests/run_npu_kernel_smoke.py:29-36;
                            tests/test_provider_integration.py:486-514)
  physical_seq_lens         reference KAT ([301,21] -> [129,21],
                            tests/test_provider_integration.py:486-514)
  QueryStatsAccumulator     closed forms ((3,4) pairs -> means 3, 4, |q| 5;
                            half-style pair layout; gate half ignored; head-shaped
                            input equals flat); float64 loop brute force
                            (tests/test_oracle_calibration.py)
  brute.slot_mapping        closed form slot = table[p // 128] * 128 + p % 128
                            (block-table arithmetic of tri/cache.py:9-15) on
                            hand-worked cases; the GPU kernel is checked against it
"""
