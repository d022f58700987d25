"""Checker package: float64 oracle (afa_oracle) and the C contract restatement (contract).

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the product package.
"""
