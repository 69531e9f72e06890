"""CPU oracle for SBDA attention -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, for the
baseline, as the timed CPU restatement).  The shipped package never imports
it: the GPU path fails loudly when its HIP library is missing instead of
falling back to anything here.

Every function in :mod:`oracle.sbda_oracle` cites the reference file:line it
restates and is pinned by tests in ``tests/test_oracle.py`` (brute-force
loops, closed forms, fp64 gradcheck, special cases and the reference's own
known answers).  No function here is "parity unpinned".
"""
