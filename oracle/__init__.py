"""CPU oracle for the FlashLog propagation hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
as the checker, and by bench.py's cpu_baseline leg.  The product package
(``flashlog_amd``) never imports this package.
"""
