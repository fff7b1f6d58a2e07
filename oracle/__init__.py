"""
ORACLE -- test infrastructure only.

CPU restatements of the reference's MoE hot path used as the checker by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg.  nanospeaker_amd/ never imports
anything from here.
"""
