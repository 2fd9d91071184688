"""CPU oracle of the Iris-3B denoise step: test infrastructure, never a product path.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this package.
"""
