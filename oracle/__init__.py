"""CPU oracle of the kernel-rsi fused kernels -- test infrastructure only (see krsi_oracle.py)."""
