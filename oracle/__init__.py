"""TEST INFRASTRUCTURE ONLY: the oracle (CPU restatement) of kern-glm53's `glm_deepgemm` path.

Imported only by tests/, `__graft_entry__.smoke()` and bench.py's `cpu_baseline` leg, to check
the product against (and, in the bench, to time the CPU baseline).
The product package never imports it.
"""
