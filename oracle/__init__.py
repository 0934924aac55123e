"""CPU oracle of FERRY's per-GPU MoE hot path -- TEST INFRASTRUCTURE ONLY.

Restatements of the reference algorithms on the CPU (numpy, torch-CPU, and C in
ref_core.c), each citing the reference file:line it follows.  Only the test suite,
``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` may import this package,
and only to check results or as the timed CPU baseline; the product (ferry_amd) never calls it.

How each function is pinned (beyond restating the reference):
  topk (ref_core.c)      -- index-for-index against torch.topk on the CPU (the library the
                             reference calls), tie-heavy rows included.
  router                 -- the reference op sequence in torch-CPU; torch.topk itself.
  history                -- closed form: score = count of e among the last min(W, seen)
                             tokens / n, checked against the ring restatement; fp32 division
                             equals the float64 mean cast to fp32 for all 0 <= c <= n <= 128.
  plan_layer (ref_core.c) -- hand-derived known-answer scenarios, a sort-based brute-force
                             formulation on random small caches, and invariants.
  layout                 -- closed form via numpy stable argsort, checked against a
                             pure-Python restatement of build_layout's loops.
  experts / combine      -- torch-CPU op order of execute_experts / reduce_partials, checked
                             against an fp64 SwiGLU and exact fp32 sums.
  shared experts         -- HF DeepseekV2MLP op order in torch-CPU bf16, checked against an
                             fp64 SwiGLU (the HF code itself is not the reference and is only
                             restated).
"""
