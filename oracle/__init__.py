"""CPU oracle of the KV-cache data path -- TEST INFRASTRUCTURE ONLY.

A NumPy restatement of the reference's (rouviere-german/paged-kv-serving, pure Python + NumPy)
algorithms on the hot path, written for this repository. Each function cites the reference
file:line it follows (paths relative to the reference repository root). It is the checker the
HIP kernels are compared against; it is never the thing measured or shipped:

* only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
  import it;
* the product package ``paged_kv_serving_amd`` never imports it and has no CPU fallback.

Modules:
    attention  -- paged online-softmax attention (attention.py:42-121) and float64 closed forms
    model      -- the fp32 decoder math and the cache-free recompute (model.py:43-288)
    runner     -- slots, append, copy-on-write and the paged forward (runner.py:95-227)
    bf16       -- round-to-nearest-even float32 -> bfloat16 for the bf16-KV tolerance oracle

Each function is pinned (closed forms, invariants, brute force on tiny inputs, planted mistakes)
by ``tests/test_oracle_*.py``.
"""
