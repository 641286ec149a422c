"""CPU oracle for the q2fp8 pruned decode path.

TEST INFRASTRUCTURE: this package is the checker, never the product.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
it.  The HIP product path in ffa-speedtest_amd/ does not import it and fails
loudly when its native library is missing.
"""
