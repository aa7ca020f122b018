"""CPU oracle for the cmpext3 GEMM path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or the timed CPU baseline), never as the
thing measured or shipped.  The product path (cmp_ext_amd) never imports it.
"""
