"""CPU oracle for the draft-objective hot path (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the reported
CPU baseline.  The product (``nanospec_amd``) never imports it and has no CPU
fallback.
"""
