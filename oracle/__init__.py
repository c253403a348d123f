"""CPU oracle for the PhaseKV Stage-B decode path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy on the host, the reference algorithms that the
HIP kernels in ``phasekv_amd`` implement:

* ``packing_oracle``       — ``src/phasekv/kernels/packing.py:26-175``
* ``attention_oracle``     — ``src/phasekv/kernels/reference.py:27-109`` and the
  split/merge math of ``src/phasekv/kernels/attention_triton.py:257-307,604-669``
* ``launch_config_oracle`` — ``src/phasekv/kernels/launch_config.py:6-64``
* ``cache_oracle``         — the hot window lifecycle of
  ``src/phasekv/phasekv_cache.py:101-114,322-340,405-422``
* ``select_oracle``        — prefill prompt selection, ``src/phasekv/prompt_tier.py:22-76``
  and ``src/phasekv/hetero_cache.py:55-94,147-157``

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker.  The product
path (``phasekv_amd``) never imports it and has no CPU fallback.

Pinning status (what checks each function independently of its own formula):

* pack_low_bits / unpack_low_bits — exhaustive brute force over every byte value
  and lengths 1..33 against a bit-by-bit construction, plus golden vectors
  written by the reference's own ``packing.py`` (tests/golden).
* quantize_pack / unpack_dequantize — golden vectors from the reference's
  ``packing.py`` (tests/golden), plus closed forms: constant groups, two-valued
  groups, exact half-way ties, a case where the fp32 and fp16 scales give
  different codes, tail groups and group size 1.
* attention (fused_decode_attention_reference, dense_fp16_attention,
  reduce/merge) — float64 brute force on tiny inputs, closed forms (uniform
  softmax, one dominant key), and invariants (segment order, split count, LSE
  merge associativity, GQA head mapping).
* cache_oracle (append, value norms, kept-token selection, cooling) — the
  selection equals torch's own ``vector_norm(...).topk(k).indices.sort()`` (the
  calls the reference makes) on tie-free inputs; norms within 1 ulp-scale of a
  float64 norm; ties and NaN by brute force over explicit rankings; the cooled
  segment equals ``quantize_pack`` of the kept rows and the shifted window equals
  slicing; ``keep_count`` against Python's round on half-way cases.  Parity unpinned:
  which of several tokens with exactly equal V norms is kept (``torch.topk`` does not
  fix it; here the earlier token).
* select_oracle (votes, pooling, kept positions) — votes, pooling and the kept set
  equal torch's own ``float().sum``, ``F.max_pool1d`` / ``F.avg_pool1d`` and
  ``topk().indices`` (the calls the reference makes) on tie-free inputs; the plan
  against hand-worked budgets; max pooling exact against a brute-force window max;
  ties and NaN by brute force.  Parity unpinned: which of several candidates with
  exactly equal pooled scores is kept (``torch.topk`` does not fix it; here the earlier
  position), and the votes' float32 summation order against torch's reduction order.
* plan_kivi_decode — known-answer tests from the reference's
  ``tests/test_phasekv_launch_config.py:10-47`` and the published plan table
  (``docs/idea/PhaseKV-技术原理与系统设计.md:495-502``).
"""
