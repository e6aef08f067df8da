"""CPU oracle package (test infrastructure only; see gdn_oracle.py)."""
