"""CPU oracle package -- test infrastructure only (see sihc_oracle's header)."""
