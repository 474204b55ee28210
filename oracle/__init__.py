"""CPU oracle for the batched sampling path (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg may
import this package, and only as the checker.  The product package
(``tachyon_amd``) never imports it.
"""
