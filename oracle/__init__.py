"""CPU oracle: a restatement of the reference's hot-path algorithms in numpy.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (`slimkv_amd/`) imports,
calls or links anything here; only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` use it, to check results and time the host.

Modules (each function cites the reference file:line it restates):
  bf16       - round-to-nearest-even bfloat16 on float arrays (bit arithmetic)
  rope       - RoPE tables and the bf16-exact decode / prefill rotations
  attention  - eager grouped attention with LSE, query absorption, V lift,
               LSE merge, the layer-level latent decode and reconstruction
  paged      - beacon/raw page index math of the paged cache
  splits     - split-count heuristics of the reference decode extension
  brute      - pure-Python loop versions used to pin the vectorised ones

How each function is pinned (golden vectors, closed forms, invariants,
brute force) is listed in tests/test_oracle_*.py.
"""
