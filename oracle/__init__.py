"""CPU oracle for the qwen4exp token-mixing path (QSA + Gated DeltaNet).

TEST INFRASTRUCTURE ONLY. This package is the checker, never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only to compute expected values or to time the
CPU baseline. The HIP path in ``ttrunner-qwen38-flash-next_amd`` never imports,
calls or falls back to anything here.

What it is: a plain PyTorch (CPU) restatement of the reference engine's
token-mixing arithmetic, op for op, so that on the same inputs it produces the
same float32/bfloat16 values as the reference module does:

* ``layers``    -- reference/layers.py primitives (norms, rope, conv, delta rules)
* ``mixing``    -- reference/model.py ``_linear_attention`` / ``_indexer_mask`` /
                   ``_full_attention`` as functions over a weight getter + cache
* ``cache``     -- reference/cache.py ``LayerCache`` / ``HybridCache``
* ``selection`` -- the integer rules of the QSA selection (eligibility, tail,
                   top-k with lower-index ties, block -> page gather), in numpy
* ``f64``       -- a float64 twin of the recurrence for tolerance analysis
* ``config``    -- the dimensions the reference derives in reference/config.py

How each function is pinned (golden vectors from the reference, closed forms,
brute force, invariants) is stated in that function's module header.
"""
