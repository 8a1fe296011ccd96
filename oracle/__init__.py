"""CPU oracle of the blockscale fused-MoE path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, as the checker; the aiter_amd product path never does.
"""
