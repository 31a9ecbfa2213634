"""CPU oracle for the EF / k-quant encoder path. TEST INFRASTRUCTURE ONLY.

This package restates the reference's algorithms on the CPU (numpy) so the HIP
kernels can be checked against them. It is a reference for tests, never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import it. The shipped path (``perm_amd``) never imports, links or falls
back to anything here.

Modules
  kquant_oracle  -- coldpress/kquant.py: k-quant encoders / decoders
  ef_oracle      -- coldpress/ef.py:46-218: inverse-Cholesky factor, committed
                    grid, code repack, the EF column sweep
  hess_oracle    -- coldpress/hessians.py:137-154: X^T X accumulation
  perm_oracle    -- coldpress/perm: Qwen3 index moves, the container objective
                    (objective.py) and the space-map optimizer (qwen3.py)
"""
