"""CPU oracle of the attention hot path.  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and
only to check results (or as the timed CPU baseline), never as part of the product path.

Contents (each function cites the reference lines it restates; nothing is imported from the
reference):
  sdpa.attention_ref     fp32 SDPA with repeat_kv and an explicit bottom-right causal mask, run
                         per row on the row's real keys: kernels/test_fa2.py:28-35,54-57 and the
                         model's CPU fallback model.py:70-75,102-107.
  sdpa.lse_ref           log-sum-exp of the scaled scores, the L the reference kernel computes
                         (kernels/fa2.py:155-158).
  sdpa.varlen_ref        the same per row of a packed batch.
  paged.gather_dense     the paged cache's slot arithmetic and dense gather (kv_cache.py:15-16,
                         93-98, 117-121).
  paged.build_pool       a KVCache-layout pool + per-row block tables from dense K/V.
  brute.attention_f64    float64 loops over (row, head, query, key): the textbook definition,
                         used to pin sdpa.attention_ref on small shapes.
  rope.apply_rope        rotate-half RoPE in the tensor dtype (model.py:58-65) and its cos/sin
  rope.rope_cos_sin      tables (model.py:151-155); rope.cache_write, the cache scatter
  rope.cache_write       (kv_cache.py:108-115).
  sample.sample          last-position sampling (chat.py:103-107) as an exponential race over
                         Philox4x32-10 uniforms (sample.philox4x32, sample.uniforms), float64.

sdpa.attention_ref, sdpa.lse_ref and brute.attention_f64 take any head dim d for Q/K and d_v for
V (the launcher's envelope, kernels/fa2.py:172,185) and any float dtype (computed in fp32 / fp64).

The seeded workload generators are not part of the oracle: they live in the package
(my-inference-engine_amd/workloads.py) because bench.py's GPU leg needs them too.

Parity status: every function above is pinned: the attention and cache functions by
tests/test_oracle.py (fp64 brute force, also with d_v != d; closed forms; GQA / permutation /
padding invariants; planted mistakes), RoPE by tests/test_rope.py, the sampler by
tests/test_sample.py (the Random123 known-answer vectors, chi-square against softmax(logits/T)).
None is "parity unpinned".
"""
