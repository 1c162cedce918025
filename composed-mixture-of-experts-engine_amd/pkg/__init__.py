"""Reference-compatible import surface (``pkg.kernels``, ``pkg.distributed``).

The reference's callers import ``pkg.kernels.moe_router`` and
``pkg.distributed.{router,moe_layer,mesh}``; this package keeps those module
paths, class names, signatures and return types, and runs every compute step
on the gfx950 kernels of ``moe_mi355``.
"""
