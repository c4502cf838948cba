"""CPU restatement of darknet-zig's CPU twins: the parity oracle.

TEST INFRASTRUCTURE ONLY -- imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product path (darknet_zig_amd).
"""
