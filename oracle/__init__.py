"""TEST INFRASTRUCTURE ONLY: the CPU oracle (see oracle.py, mla_oracle.c)."""
