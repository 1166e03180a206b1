"""CPU restatement of the reference's hot-path algorithm -- test infrastructure only.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker.
The product (moa-workspace_amd/) never imports it.
"""
