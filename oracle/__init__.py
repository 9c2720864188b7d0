"""CPU oracle for the ASPA forward path (test infrastructure only).

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
as the checker; never by the proteus_attention product package.
"""
