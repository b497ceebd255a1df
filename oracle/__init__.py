"""Test infrastructure only: CPU restatement of the reference's CPU-fallback semantics.

Nothing in the product (the ``pytorch-apple_amd`` package) imports this package;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, always as the checker.
"""
