"""Test infrastructure: CPU oracles for the paged decode path.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import anything here, and only as the checker or the reported CPU
baseline; the product path never does.
"""
