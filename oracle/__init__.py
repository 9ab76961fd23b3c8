"""CPU oracle for the sampler -- test infrastructure only (see oracle/oracle.py)."""
