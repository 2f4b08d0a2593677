"""Test infrastructure: CPU restatement of Flare's sparse-embedding hot path.

Nothing in the product imports this package.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it,
and only to check results (or, for ``bench.py``, as the timed CPU baseline).
"""
