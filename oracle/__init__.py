"""CPU oracle for the pruned-weight MatMul/Gemm path.

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU
baseline, never as the product.  The product package (pyflamert_amd) never
imports it.
"""
