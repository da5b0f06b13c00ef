"""Test infrastructure: the CPU oracle of the DSA decode path (dsa_oracle). Imported only by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker; never by trnrt_amd."""
