"""CPU oracle for the selective-scan hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithms the MI355X kernels must reproduce:

* ``ssm_ref.selective_scan_ref`` -- torch restatement of ``selective_scan_ref``
  (reference ``mamba_ssm/ops/selective_scan_interface.py:353-451``), real-A / non-P/Q part.
* ``ssm_ref.selective_state_update_ref`` -- the single-token decode update
  (reference in-tree math ``mamba_ssm/modules/mamba_simplemotif.py:369-376``; upstream
  ``mamba_ssm.ops.triton.selective_state_update`` 2.2.6.post3, not vendored).
* ``brute`` -- pure-Python float64 closed-sum restatement for tiny shapes (independent of the
  recurrence form: h_t = sum_k prod_{j>k} a_j * b_k).
* ``scan_f64.c`` -- C float64 sequential restatement, OpenMP over rows, used to check sampled
  rows at the full benchmark shapes (built by ``__graft_entry__.build()`` with gcc into
  ``oracle/_build/``; the reference itself is CUDA/pybind and is not built here).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker / the timed CPU baseline. The product path
(``motif-mamba_amd/``) never imports it and fails loudly when its HIP library is missing.

Pinning status of each function is recorded in the module docstrings and in ``tests/test_oracle.py``.
"""
