"""CPU oracle for the paged-attention hot path (test infrastructure only).

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker.  The product package flexengine_amd never imports it.
"""
