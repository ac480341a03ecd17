"""CPU oracle for the `@parallel` path: TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package.  The shipped ``lcd_amd`` package never
does; it fails loudly when its HIP library is missing instead.
"""
