"""ORACLE — test infrastructure, not product code (see ebag_oracle.py)."""
