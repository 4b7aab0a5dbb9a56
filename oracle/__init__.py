"""CPU oracle of the key-scan path: test infrastructure only (see fathom_oracle)."""
