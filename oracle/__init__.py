"""CPU oracle of the rotor ternary-linear path -- TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, always
as the checker (or the timed CPU baseline); never by the product package.
"""
