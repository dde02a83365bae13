"""TEST INFRASTRUCTURE ONLY: the parity oracle of the attention forward path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker; pmkl_amd/ never does.
"""
