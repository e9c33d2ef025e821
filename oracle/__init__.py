"""CPU oracle for the packed-trit fabric -- test infrastructure only (see oracle.py)."""
