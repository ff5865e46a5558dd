"""CPU oracle of the MXFP4 path — test infrastructure only (see oracle/mxoracle.h)."""
