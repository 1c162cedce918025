"""The C-ABI library loads on a CPU host, exports every symbol the header
declares, and rejects bad arguments before touching the GPU (CPU only: no
call here launches a kernel)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from moe_mi355 import _lib

pytestmark = pytest.mark.cpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "moe_mi355.h")


def _declared_functions():
    with open(HEADER) as f:
        src = f.read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(moe_\w+)\s*\(", src, flags=re.M)
    return sorted(set(names))


def test_library_built():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() first"


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    declared = _declared_functions()
    assert declared, "header parse found no functions"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/moe_mi355.h but not exported"
    assert sorted(_lib.exported_symbols()) == declared


def test_version_string():
    assert b"gfx950" in _lib.load().moe_version()


def test_router_fwd_rejects_bad_shapes_without_gpu():
    lib = _lib.load()
    # K > E
    rc = lib.moe_router_fwd(None, 1, None, 1, None, 16, 64, 4, 8, None, None, 1, None, None, None, None, 0.0, 0.0, None, None, None, 0, None)
    assert rc == -1
    assert "bad shape" in _lib.last_error()
    # unsupported dtype code
    rc = lib.moe_router_fwd(None, 7, None, 1, None, 16, 64, 8, 2, None, None, 1, None, None, None, None, 0.0, 0.0, None, None, None, 0, None)
    assert rc == -1 and "dtype" in _lib.last_error()
    # null pointers
    rc = lib.moe_router_fwd(None, 1, None, 1, None, 16, 64, 8, 2, None, None, 1, None, None, None, None, 0.0, 0.0, None, None, None, 0, None)
    assert rc == -1 and "null" in _lib.last_error()


def test_router_bwd_rejects_bad_shapes_without_gpu():
    lib = _lib.load()
    rc = lib.moe_router_bwd(None, 1, None, 1, None, None, None, 1, None, None, None, 0.0, 0.0,
                            16, 64, 300, 2, None, None, None, 0, None)
    assert rc == -1 and "bad shape" in _lib.last_error()


def test_workspace_queries_are_pure_host_arithmetic():
    lib = _lib.load()
    a = lib.moe_router_fwd_workspace(16384, 4096, 8, 2, 1, 1)
    b = lib.moe_router_bwd_workspace(16384, 4096, 8, 2, 1, 1)
    assert a > 0 and b > 0
    assert lib.moe_router_fwd_workspace(0, 4096, 8, 2, 1, 1) == 0


def test_check_raises_value_error_for_argument_codes():
    lib = _lib.load()
    rc = lib.moe_router_fwd(None, 1, None, 1, None, 16, 64, 4, 8, None, None, 1, None, None, None, None, 0.0, 0.0, None, None, None, 0, None)
    with pytest.raises(ValueError):
        _lib.check(rc, "moe_router_fwd")


def test_cpu_tensors_are_rejected_not_routed_to_a_fallback():
    import torch

    from moe_mi355 import ops

    with pytest.raises(RuntimeError, match="GPU"):
        ops.router_forward(torch.zeros(4, 8), torch.zeros(8, 4), 2)


def test_torch_binding_loads_and_shares_the_library():
    """moe_mi355/_moe_torch.so (the router's C++ autograd Function) imports, links the in-tree
    libmoe_mi355.so, and its entry point rejects CPU tensors through RouterCore's checks."""
    import torch

    from moe_mi355 import router as R

    mod = R._binding()
    assert os.path.dirname(os.path.abspath(mod.__file__)) == os.path.dirname(os.path.abspath(_lib.LIB_PATH))
    assert callable(mod.router_core)
    with open("/proc/self/maps") as f:
        maps = f.read()
    assert os.path.realpath(_lib.LIB_PATH) in maps
    with pytest.raises(RuntimeError, match="AMD Instinct GPU"):
        R.RouterCore.apply(torch.zeros(4, 8), torch.zeros(8, 2), 1, 0.0, 0.0, None)
