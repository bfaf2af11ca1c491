"""CPU oracle of the W4A4 path -- test infrastructure only.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import this package; the product (``pi05_fast.w4a4``) never does.
"""
