"""CPU oracle of the relative_key attention path -- test infrastructure only.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker; the product path never imports it.
"""
