"""CPU oracle of the attention forward -- test infrastructure, not product code.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg. See oracle/attention.py for what each function restates and what pins it.
"""
