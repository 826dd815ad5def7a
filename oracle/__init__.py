"""Oracle for the decode hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU leg (the CPU
baseline, and the check of every timed op's output before it is timed) import
this package, and only as the checker (or, for the CPU baseline, as the
reference's CPU path being timed). The product (``decodekernels_amd``) never
imports it and has no CPU fallback: without the HIP libraries its ops raise.

* ``oracle.reference`` -- CPU restatement of DecodeKernels'
  ``decode_kernels/reference.py`` (same function names and signatures, torch on
  the CPU in fp32), the expected results of every op.
* ``oracle.brute`` -- independent float64 numpy brute force on tiny inputs,
  written from the definitions (softmax attention with GQA head mapping
  ``kv_head = q_head // group``, the log-sum-exp merge, ``A·Bᵀ``, RMSNorm,
  SiLU), used to pin ``oracle.reference``.
* ``oracle.rope_cache`` -- rotary embedding and the paged cache write, the
  two steps around attention that DecodeKernels leaves to vLLM, restated from
  their published definitions; pinned in ``tests/test_oracle_rope_cache.py``
  (complex-multiplication route, rotation invariants, ``index_put_`` scatter,
  planted mistakes).

Pins (see ``tests/test_oracle.py``): every function of ``oracle.reference`` is
checked against ``oracle.brute`` and against a torch library routine or
closed form (``F.scaled_dot_product_attention``, ``F.linear``, ``F.silu``,
``x / sqrt(mean(x^2) + eps) * w``), and the reference's own CPU properties
(``tests/test_reference.py:30-124``: split-K merge == dense at partition
boundaries, paged gather == contiguous attention for block sizes 1/16/32,
strided HND / vLLM views == contiguous copies, empty sequences -> zeros,
residual rounding). Planted mistakes in the oracle (dropped scale, wrong GQA
mapping, transposed operand, unweighted merge, unrounded residual) are shown
to fail at least one pin. The reference ships no golden vectors or fixtures.
"""
