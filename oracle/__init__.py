"""CPU oracle for the fp32 GEMM hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this package, and only as the checker or the timed CPU baseline.
The product package (``zigneuron_amd``) never imports it.
"""
