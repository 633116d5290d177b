"""CPU oracle of the attention hot path — TEST INFRASTRUCTURE ONLY (see oracle.c's header).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package.
"""
