"""TR-MoE CPU oracle -- test infrastructure only (see trmoe_oracle.py)."""
