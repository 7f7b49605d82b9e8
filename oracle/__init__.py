"""CPU oracle for the MI355X backend — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU with numpy, what the reference computes on the
hot path: the index maps of arranged tensors (``arrange``) and the six applications
executed tile by tile over those maps (``apply``).  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import
it, and only as the checker or the reported CPU baseline; the product package
``ninetoothed_amd`` never imports it and has no CPU fallback.

What pins each part (details in each module's docstring):
  - arrange: the reference's literal golden maps (tests/golden/index_maps.json,
    transcribed from the reference's tests/test_debugging.py and tests/test_eval.py)
    and hand-checkable closed forms of tile/expand/permute/flatten/pad;
  - apply: torch closed forms at small shapes (matmul, addmm, conv2d, scaled dot-product
    attention, softmax, max_pool2d, add) in float64/float32, invariants (softmax rows
    sum to 1, attention with one key returns v, causal row 0 returns v[0]) and
    brute-force loops on tiny shapes.
"""
