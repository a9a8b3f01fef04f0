"""CPU oracle (test infrastructure only; see sdpa_oracle.py)."""
