"""CPU oracle for the compressed-KV hot path — test infrastructure only (see cpu_ops.py).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package;
the kushkash_amd product path never does."""
