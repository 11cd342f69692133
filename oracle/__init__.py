"""CPU oracle for rabbit_amd: a restatement of ferrumox/rabbit's routed-expert path.

TEST INFRASTRUCTURE ONLY -- imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg as the checker and the CPU baseline; never by the product (rabbit_amd).
"""
