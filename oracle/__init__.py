"""CPU oracle for the Q4 dequant-matvec path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, as the checker; the product library never does.
"""
