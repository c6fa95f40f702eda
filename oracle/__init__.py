"""Oracle (test infrastructure only): CPU restatements of the reference's golden path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only to check results.  The product (ffn_optim_amd/) never
imports it and has no CPU fallback.
"""
