"""CPU oracle package - test infrastructure only (see o1_oracle.h)."""
