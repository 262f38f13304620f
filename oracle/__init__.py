"""The CPU oracle of the hsd hot path (test infrastructure only; see hsd_oracle)."""
