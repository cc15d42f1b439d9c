"""CPU oracle for tilec's matmul path — test infrastructure only (see oracle.py)."""
