"""CPU oracle for the attention + speculative-verify hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this package:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and there only as the checker (or the timed CPU baseline),
never as the computation under test.

Each function restates the reference algorithm on the CPU with PyTorch fp32 (or
plain integer indexing), citing the reference file:line it follows:

* ``kvcache.store_kvcache``            nanovllm/layers/attention.py:10-40
* ``attention.paged_decode_attention`` nanovllm/layers/attention.py:71-78
  (flash_attn_with_kvcache, bottom-right causal, paged KV)
* ``attention.varlen_attention``       nanovllm/layers/attention.py:64-70
  (flash_attn_varlen_func, optional block_table)
* ``sampler.verify_drafts``            nanovllm/layers/sampler.py:28-103
* ``sampler.chunked_logsumexp``        nanovllm/layers/sampler.py:19-25
* ``sampler.sample``                   nanovllm/layers/sampler.py:5-16

How each one is pinned (checked independently of its own formula) is listed in
``tests/test_oracle.py``:

* store_kvcache: brute-force per-row loop, -1 skip, bit-exact.
* attention: textbook SDPA (torch.nn.functional.scaled_dot_product_attention
  with an explicit boolean mask) on gathered pages; single-block and n=1 special
  cases; a planted-value test that fails on a wrong GQA head mapping, a wrong
  causal offset or a wrong block-table lookup; varlen == decode on the same
  sequences.
* verify_drafts: the reference unit tests' known answers (greedy), its
  total-variation-distance test and zero-residual guard, and golden vectors
  written by the reference's own sampler.py (tests/golden/).
* sample: closed form on tiny inputs (greedy rows equal argmax; random rows
  equal argmax of p / max(E, 1e-10)) and the TV-distance property.
"""
