"""CPU oracle for the LUCID attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithm on the CPU in float64 (numpy /
scipy) so that the HIP kernels in ``lucid_amd`` can be checked against it.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed CPU baseline.
The product path (``lucid_amd``) never imports anything from here and fails
loudly when its HIP library is missing.

Modules
-------
lucid_ref  -- LUCID preconditioned attention (modeling_lucid.py) in float64,
              plus a float32 torch restatement of the reference's dense path
              used as the CPU baseline.
path_ref   -- LUCID-Path (lucid_path/triton_code) brute force and chunked
              restatements in float64.

Pinning (how each oracle function is itself checked) is recorded in the
docstring of every function and exercised by ``tests/test_oracle_*.py``.
"""
