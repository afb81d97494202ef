"""CPU oracle for the paged-KV hot path — TEST INFRASTRUCTURE ONLY.

A restatement of the reference's algorithm (src/helios/runtime/qwen3/paged_cache.py,
cache.py, layers.py) used to CHECK the HIP kernels. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import
it. Nothing in the ``helios_amd`` package imports it, and it never stands in for a
kernel.

Modules
  attention   float64 numpy restatement of paged varlen GQA attention
              (paged_cache.py:378-414, :521-546 and the varlen_attn call contract at
              :316-329, :506-519).
  dense_torch the reference's own dense-KV CPU path, op for op in torch fp32
              (index_select gather, repeat_interleave, SDPA with a bool mask); the
              timed CPU baseline.
  kv_bytes    numpy restatements of the bit copies: KV append (index_copy_,
              paged_cache.py:335-345), page gather (_gather_cpu, :405-414) and block
              copy (cache.py:109-147).

How each function is pinned (tests/test_oracle.py): against closed forms
(L = 1 gives V[0]; equal keys give the mean of V; a dominant key selects its V row;
a fresh causal prefill equals the textbook lower-triangular softmax), brute-force
pure-Python loops on tiny inputs, torch's own index_copy_ / index_select /
scaled_dot_product_attention, invariance under permutation of physical pages, the
known-answer metadata values of the reference's tests, and the committed golden
fixtures in tests/golden/.
"""
