"""Oracle for value projection + multi-scale deformable attention. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, and only as the checker
(or as the timed CPU baseline); the product (marearts_tinydeform_amd) never imports, calls or links it.

  oracle.bruteforce   float64 numpy restatement of the reference's corner rule and weighted sum
  oracle.gridsample   torch restatement of the reference's PyTorch path (F.linear + grid_sample per level), and
                      the gradient oracle of the backward (PyTorch autograd through it in float64)

Pinning: see tests/test_oracle.py (grid_sample agreement, closed forms, invariants, planted mistakes, golden
fixtures) and tests/test_backward.py (gradients against central finite differences of the brute force). The reference repository ships no golden vectors, so no reference-held fixture exists to check against.
"""
