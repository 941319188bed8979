"""CPU oracles of the LSSO mixer.  Test infrastructure only: imported by
tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg, never by the
lsso_amd package."""
