"""CPU oracle package -- test infrastructure only (see mlp_oracle.py)."""
