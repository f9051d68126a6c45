"""CPU oracle for the compact-DMS hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (integer/byte work) and numpy/torch-CPU float
arithmetic, what shisa-ai/FastDMS computes on its compact-DMS path.  Every
function cites the reference file:line it follows.  It is the checker that the
HIP kernels in ``fastdms_amd`` are compared against, and the CPU baseline that
``bench.py`` times beside the GPU.

Rules this package obeys:

* Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
  ``bench.py`` may import it.  ``fastdms_amd`` never imports it; the product
  path raises if its HIP library is missing instead of falling back here.
* Each function is pinned by the reference's literal vectors (``tests/golden``),
  by a library routine (torch's own FP8 cast, numpy softmax in float64), or by
  a mathematical invariant tested in ``tests/test_oracle_*.py``.  Functions with
  no such pin are marked "parity unpinned" in their docstring.
"""
