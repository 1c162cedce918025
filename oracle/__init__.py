"""CPU oracle for the MoE hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU and in float64 (torch) / integer numpy, the
algorithm of the reference moe-engine hot path:

* ``oracle.router``  -- top-k router forward/backward, dispatch counts,
  load-imbalance, z-loss, and the load-balance aux loss / differentiable
  z-loss (closed forms; absent from the reference).
* ``oracle.plan``    -- ``_cumcount``, the per-top-k-column capacity drop mask,
  the reference "positional" layout and the routed layout.
* ``oracle.layer``   -- the SwiGLU expert and the full MoE layer forward /
  backward in both layouts.
* ``oracle.norm``    -- the RMSNorm in front of the router and its backward.
* ``oracle.fp8``     -- the e4m3 row quantization and the fp8 expert forward
  (this build's own variant: the reference has no fp8 path).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker (or the timed CPU
baseline).  The product (``moe_mi355`` / ``pkg``) never imports it: on a
machine without the HIP library the product raises instead of falling back
here.

Every function cites the reference file:line it restates
(paths relative to the reference's ``moe-engine/`` directory).

Pinning status (what checks each function against something other than
itself) is listed in each module's header.
"""
