"""CPU oracle of the beam search (test infrastructure only; see bs_oracle.c)."""
