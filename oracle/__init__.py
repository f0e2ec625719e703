"""Oracle for the paged-KV data plane -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

A CPU restatement of the reference's torch path for the paged-KV hot path
(src/mini_infra/worker/paged_kv_cache.py, src/mini_infra/worker/paged_runner.py,
src/mini_infra/model/qwen3.py), used only as the reference the tests compare against:

* ``oracle.torch_ref`` -- the reference's op chains (advanced-index gather, index_copy_,
  repeat_interleave, bf16 matmul, fp32 softmax) in the same order with the same bf16
  rounding points, on CPU tensors.  It is also the CPU baseline the benchmark times.
* ``oracle.closed_form`` -- independent statements of what the mathematics fixes: the
  scatter/gather index identities in numpy, and fp64 brute-force attention with explicit
  loops.  Tests pin ``torch_ref`` against these and against the known-answer tests of the
  reference's own suite before trusting it.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import
this package.  The product (``mini_infra_qwen3_amd``) never does: it has no CPU path.
"""
