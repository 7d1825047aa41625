"""CPU oracle of the Engram lookup path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as the expected result the HIP path is tested against (or as the timed CPU baseline).
The product package never imports it.

Contents (each function cites the reference code it restates):
  hash_oracle.c / engram.py   mults, hash_ids, hash_prev (integer, bit-exact)
  engram.py                   lookup, inject (torch CPU fp32 op-for-op), dedup (numpy),
                              rowwise LazyAdamW + stochastic bf16 rounding, Philox4x32-10

Pinning (what checks each function against something other than itself) is listed in the
header of engram.py and exercised by tests/test_oracle_*.py.
"""
from .engram import *  # noqa: F401,F403
