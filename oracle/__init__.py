"""TEST INFRASTRUCTURE ONLY: the oracle (CPU restatement) of kern-glm53's `glm_deepgemm` path.

Imported only by tests/, `__graft_entry__.smoke()` and bench.py's `cpu_baseline` leg, as the checker.
The product package never imports it.
"""
