"""CPU oracle (test infrastructure only): see ``oracle/oracle.py``.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package; the shipped ``looped_blockell`` path never does.
"""
