"""CPU oracle for the paged-attention hot path.

TEST INFRASTRUCTURE ONLY. It restates, on the CPU, the reference algorithms
this repository's kernels must reproduce:

* ``attention``: CpuAttentionBackend (src/core/attention_backend.py:56-144),
  its GQA extension (transformers' repeat_kv grouping as used at
  src/core/model_adapter.py:506-507), the partial-softmax merge of
  src/core/resident_kv_store.py:2497-2509, and chunked prefill defined as
  successive append-then-attend decode steps;
* ``blocks``: KVCacheManager's block bookkeeping
  (src/core/memory_manager.py:55-173).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the reference results a
test compares against or as the timed CPU baseline. The product package ``cloverinfer_amd`` never imports it.

Every function is pinned by checks in tests/test_oracle.py that do not
retype its formula: the reference tests' known answers
(tests/golden/reference_kats.json), closed forms (uniform and one-hot
softmax), float64 brute force on tiny shapes, and invariants (split-K
partition independence, GQA == repeat_kv expansion, chunked prefill ==
successive decode steps).
"""
