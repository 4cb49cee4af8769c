"""CPU oracle of HyMT2Sharp's attention path.

TEST INFRASTRUCTURE ONLY (see hymt_oracle.h): imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product.
"""
