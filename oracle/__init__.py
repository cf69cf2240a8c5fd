"""CPU oracle for the 4-bit dequant matmul path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package; the shipped library never does.
"""
