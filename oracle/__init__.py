"""CPU oracle of the decode-matmul path (test infrastructure only; see oracle/oracle.py)."""
