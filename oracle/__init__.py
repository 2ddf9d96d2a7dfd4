"""CPU oracle for the fused GEMM+epilogue path — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
import this package, and only as the checker or as the timed CPU reference.
The product (``fuseml_amd``) never imports it.
"""
