"""CPU oracle of the decode hot path -- TEST INFRASTRUCTURE ONLY.

Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
as the checker or the timed CPU baseline; the product never imports it.
"""
