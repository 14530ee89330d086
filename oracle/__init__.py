"""CPU oracle for the complexity-deep hot path — TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as
the checker.  The product never imports it.  See oracle/oracle.py.
"""
