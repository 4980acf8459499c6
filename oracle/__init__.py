"""TEST INFRASTRUCTURE ONLY: CPU parity oracle (see oracle/reference.py)."""
