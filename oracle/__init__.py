"""CPU oracle (test infrastructure only; never imported by trinix_amd)."""
