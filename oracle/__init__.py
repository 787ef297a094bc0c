"""CPU restatement of the Mamba SSM forward path -- test infrastructure only (see oracle.py)."""
