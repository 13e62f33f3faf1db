"""CPU oracle for the MXFP4 MoE path — test infrastructure only (see oracle.py)."""
