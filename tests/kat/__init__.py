"""Known-answer harness of the fp8 MFMA instruction (test infrastructure; see kg_mfma_kat.hip)."""
