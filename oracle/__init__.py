"""CPU oracle for the HBA forward path -- test infrastructure only (see hba_oracle.py)."""
