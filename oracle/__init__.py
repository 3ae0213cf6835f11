"""CPU oracle for the LazyRecall KV-management hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (and torch-CPU for the reference's own CPU math path), the
algorithm of every operation the HIP library implements, each function citing the reference
file:line it follows. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it, and only as the checker or as the timed CPU baseline —
never as a product code path. ``code_for_iclr27_amd`` never imports this package.

Modules:
  bf16        bit-exact bfloat16 rounding helpers (round-to-nearest-even)
  kv_ops      data movement: compact, append, legacy append/compact, merge, pack, batch_append,
              pool, merge_plan
  scoring     temporal probabilities / risk / fused head scores / legacy decision risk
  selection   refine_arrays with canonical (value, index) ties and with CPU torch.topk
  cpu_path    torch-CPU restatement of the reference CPU math path (timed CPU baseline)
  history     the query-history deques and their per-layer concatenation
  attention   causal grouped-query attention over the packed ragged layout (f64)
  vjp         head logits, one-vs-rest margins and their hidden / pre-projection gradients

How each part is pinned (checked against something other than itself) is listed in the test
files under tests/ that exercise it; see tests/test_oracle_*.py.
"""
