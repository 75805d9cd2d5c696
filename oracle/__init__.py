"""fp64 CPU oracle for the scan hot path -- test infrastructure only.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline
leg of ``bench.py``; never by the ``mingru_amd`` package.
"""
