"""CPU oracle for the AWQ W4A16 dequant-GEMM path (test infrastructure only).

Nothing in the product package imports this package. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it,
and only as the checker (or, for ``bench.py``, as the timed CPU baseline).
"""
