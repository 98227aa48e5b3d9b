"""CPU oracle of the fused EGNN/MPNN layer -- test infrastructure only.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only to check or time against it.
"""
