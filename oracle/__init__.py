"""CPU parity oracle for the MRSA hot path -- test infrastructure only.

Importable only from tests/, __graft_entry__.smoke() and bench.py's CPU
baseline leg.  See mrsa_oracle.py.
"""
