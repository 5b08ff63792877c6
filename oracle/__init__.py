"""CPU oracle of the BF16 matmul hot path -- test infrastructure, never product code.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import
it. See ``reference.py`` for the restatement and the reference lines each function follows.
"""
