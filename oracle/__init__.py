"""CPU oracle for the W8A8 MoE-FFN path: TEST INFRASTRUCTURE ONLY (see oracle.py / cb_oracle.c)."""
