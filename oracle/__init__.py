"""CPU oracle of the flat-HTRC operator -- TEST INFRASTRUCTURE ONLY.

Restatements of the reference algorithm, used solely as the checker:

* ``flat_i8``   -- ctypes wrapper of ``flat_i8.c``: the INT8 Q/K path
  (h3/htrc_flat.py:181-276 with h3/htrc_flat_triton.py:41-299), stage by stage.
* ``flat_fp32`` -- NumPy restatement of the torch backend ``_flat``
  (h3/htrc_flat.py:279-388), the reference's CPU path; timed as the CPU baseline.
* ``htrc_ref``  -- NumPy restatement of the float64 teaching reference
  (src/htrc_reference/model.py:29-137), BASELINE configuration 1, and the
  closed-form cross-check of the leaf statistics.
* ``bf16``      -- bit-level bf16 helpers shared by the above.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package.  The product package ``htrc_amd`` never
imports it and fails loudly when its HIP library is missing.
"""
