"""CPU oracle for the W8A16 decode GEMM (test infrastructure only; see oracle/oracle.py)."""
