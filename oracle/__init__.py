"""Parity oracle -- test infrastructure, not product code.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or the timed CPU
baseline). See ``morpho_oracle.py`` for what it restates and how it is pinned.
"""
