"""CPU oracle (test infrastructure only): see oracle/palu_oracle.py."""
