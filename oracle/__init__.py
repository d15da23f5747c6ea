"""CPU oracle for the decoder hot path -- test infrastructure only (see oracle.py)."""
