"""CPU oracle (test infrastructure only; see csr_oracle.py)."""
