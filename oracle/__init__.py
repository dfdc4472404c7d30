"""CPU oracle for the quantized-matmul path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package.  It is the checker the HIP kernels are compared against and is
never on the product path (edgerunner_amd does not import it).
"""
