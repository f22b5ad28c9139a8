"""CPU oracle of the draft-tree verify hot path: TEST INFRASTRUCTURE, NOT PRODUCT CODE.

This package restates, on the CPU, what the reference's kernels compute, one function per reference kernel, each
citing the reference file:line it follows (paths are relative to the eagle-harness 0.1.5 checkout). It exists to
check the HIP kernels of ``eagle-4_amd/``: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or as the timed CPU baseline. The product path never imports,
calls or falls back to anything here.

Modules:

==================  ==============================================================================================
``tables``          verify stage (depths, window codes, ancestor masks, positions), link -> parent derivation,
                    path table, tail-mask words
``conv``            width-4 tree causal conv1d with windows and the state roll
``recurrence``      gated delta rule tree walk (snapshot contract)
``records``         replay records, accepted-path commit and the parallel chunk form (records contract)
``attention``       dense tree-verify attention over a paged cache, fp8-e4m3 quantize / dequantize
``accept``          greedy tree accept walk, bs1 accept tail, row compaction, first-index argmax
``commit``          vLLM linear-state commit (window compaction, accepted state move)
==================  ==============================================================================================

Parity pins: every function is checked in ``tests/test_oracle_*.py`` against the reference tests' known answers
(masks of ``[-1, 0, 0, 1, 1, 2, 3]``, planted accept paths), independent closed forms (ancestor-bit brute force,
chain folds, links round trips) and library routines (``torch.nn.functional.scaled_dot_product_attention``).
"""
