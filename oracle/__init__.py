"""CPU oracle of the verification path — TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker or as the timed CPU baseline.  The product package ``mvsd`` never imports it.
"""
