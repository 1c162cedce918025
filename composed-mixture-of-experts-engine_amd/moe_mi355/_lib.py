"""ctypes binding of libmoe_mi355.so (the C ABI in include/moe_mi355.h).

The library is loaded lazily on first use.  A missing library or a non-ROCm
device raises immediately: there is no CPU fallback in the product path.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmoe_mi355.so")

MOE_F32 = 0
MOE_BF16 = 1
STATS_HEAD = 8

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes)
_SIGNATURES = {
    "moe_version": (ctypes.c_char_p, []),
    "moe_last_error": (_I32, [ctypes.c_char_p, _SZ]),
    "moe_prof_enable": (_I32, [_I32]),
    "moe_prof_summary": (_I32, [ctypes.c_char_p, ctypes.POINTER(_I64), ctypes.POINTER(ctypes.c_double)]),
    "moe_prof_kernel_name": (_I32, [_I64, ctypes.c_char_p, _SZ]),
    "moe_prof_mfma_ceiling": (_I32, [_I64, _I32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    "moe_prof_hbm_ceiling": (_I32, [_I64, _I32, ctypes.POINTER(ctypes.c_double)]),
    "moe_router_fwd_workspace": (_SZ, [_I64, _I64, _I64, _I64, _I32, _I32]),
    "moe_router_fwd_lds_bytes": (_I64, [_I64, _I64, _I64, _I32, _I32]),
    "moe_router_fwd": (
        _I32,
        [_P, _I32, _P, _I32, _P, _I64, _I64, _I64, _I64, _P, _P, _I32, _P, _P, _P, _P, _F32, _F32, _P, _P, _P, _SZ,
         _P],
    ),
    "moe_router_bwd_workspace": (_SZ, [_I64, _I64, _I64, _I64, _I32, _I32]),
    "moe_router_bwd": (
        _I32,
        [_P, _I32, _P, _I32, _P, _P, _P, _I32, _P, _P, _P, _F32, _F32, _I64, _I64, _I64, _I64, _P, _P, _P, _SZ, _P],
    ),
    "moe_router_bwd_acc": (
        _I32,
        [_P, _I32, _P, _I32, _P, _P, _P, _I32, _P, _P, _P, _F32, _F32, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _SZ,
         _P],
    ),
    "moe_plan_workspace": (_SZ, [_I64, _I64, _I64]),
    "moe_plan": (_I32, [_P, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "moe_plan_noalloc": (_I32, [_P, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P, _P]),
    "moe_cumcount_workspace": (_SZ, [_I64]),
    "moe_cumcount": (_I32, [_P, _I64, _P, _P, _SZ, _P]),
    "moe_permute": (_I32, [_P, _I64, _P, _P, _I64, _I64, _I64, _P, _P]),
    "moe_combine": (_I32, [_P, _I32, _P, _I32, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P]),
    "moe_combine_bwd": (_I32, [_P, _P, _I32, _P, _I32, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "moe_unpermute_sum": (_I32, [_P, _P, _I32, _P, _P, _I64, _I64, _I64, _I64, _P, _P]),
    "moe_rmsnorm_fwd": (_I32, [_P, _I32, _P, _I32, _F32, _I64, _I64, _P, _P, _P]),
    "moe_rmsnorm_router_fwd_workspace": (_SZ, [_I64, _I64, _I64, _I64, _I32, _I32]),
    "moe_rmsnorm_router_fwd": (
        _I32,
        [_P, _I32, _P, _I32, _F32, _P, _I32, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I32, _P, _P, _P, _P,
         _F32, _F32, _P, _P, _P, _SZ, _P],
    ),
    "moe_rmsnorm_bwd_workspace": (_SZ, [_I64, _I64]),
    "moe_rmsnorm_bwd": (_I32, [_P, _I32, _P, _I32, _P, _P, _P, _I64, _I64, _P, _P, _P, _SZ, _P]),
    "moe_rmsnorm_router_bwd_workspace": (_SZ, [_I64, _I64, _I64, _I64, _I32, _I32]),
    "moe_rmsnorm_router_bwd": (
        _I32,
        [_P, _I32, _P, _I32, _P, _P, _P, _I32, _P, _P, _P, _I32, _P, _P, _P, _F32, _F32, _P, _I64, _I64, _I64, _I64,
         _P, _P, _P, _P, _SZ, _P],
    ),
    "moe_quant_rows_fp8": (_I32, [_P, _I32, _I64, _I64, _I64, _P, _P, _P]),
    "moe_permute_fp8": (_I32, [_P, _I32, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "moe_swiglu_fwd_fp8_workspace": (_SZ, [_I64, _I64, _I64]),
    "moe_swiglu_fwd_fp8": (
        _I32, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _SZ, _P]
    ),
    "moe_telemetry_fields": (_I32, []),
    "moe_telemetry_record": (_I32, [_P, _I64, _I64, _I64, _F32, _P, _I64, _P, _I64, _P]),
    "moe_swiglu_workspace": (_SZ, [_I64]),
    "moe_swiglu_f32_workspace": (_SZ, [_I64]),
    "moe_swiglu_fwd_f32": (_I32, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _SZ, _P]),
    "moe_swiglu_bwd_f32": (
        _I32,
        [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _SZ, _P],
    ),
    "moe_swiglu_fwd": (_I32, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _SZ, _P]),
    "moe_swiglu_bwd": (
        _I32,
        [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _SZ, _P],
    ),
}

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def exported_symbols():
    return list(_SIGNATURES)


def load() -> ctypes.CDLL:
    """Load libmoe_mi355.so and declare every exported signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run __graft_entry__.build() "
                    "(or python moe_mi355/build.py) on a host with ROCm/hipcc"
                )
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def last_error() -> str:
    buf = ctypes.create_string_buffer(512)
    load().moe_last_error(buf, 512)
    return buf.value.decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = last_error()
        if rc < 0:
            raise ValueError(f"{what}: {msg} (code {rc})")
        raise RuntimeError(f"{what}: {msg} (hip error {rc})")


def prof_enable(on: bool) -> None:
    """Start (and clear) or stop per-kernel hipEvent timing inside the library."""
    load().moe_prof_enable(1 if on else 0)


def prof_summary() -> dict:
    """{kernel name: (launches, total ms)} for the launches recorded since prof_enable(True)."""
    lib = load()
    out = {}
    buf = ctypes.create_string_buffer(256)
    i = 0
    while lib.moe_prof_kernel_name(i, buf, 256):
        name = buf.value.decode()
        n = _I64(0)
        ms = ctypes.c_double(0.0)
        check(lib.moe_prof_summary(name.encode(), ctypes.byref(n), ctypes.byref(ms)), "moe_prof_summary")
        out[name] = (int(n.value), float(ms.value))
        i += 1
    return out


def prof_mfma_ceiling(iters: int = 100000, fp8: bool = False, random: bool = False) -> tuple:
    """(TFLOP/s, shader MHz) of a memory-free MFMA loop on every CU of the current device; ``random`` feeds
    it changing, random-looking operands (as a data-carrying GEMM does) instead of near-constant ones."""
    tf, mhz = ctypes.c_double(0.0), ctypes.c_double(0.0)
    mode = (1 if fp8 else 0) | (2 if random else 0)
    check(load().moe_prof_mfma_ceiling(int(iters), mode, ctypes.byref(tf), ctypes.byref(mhz)),
          "moe_prof_mfma_ceiling")
    return float(tf.value), float(mhz.value)


def prof_hbm_ceiling(nbytes: int, mode: int) -> float:
    """GB/s moved by a plain stream on the current device: mode 0 read, 1 write, 2 copy, 3 fan-out (each 4 KB row
    read once, written 6 times)."""
    g = ctypes.c_double(0.0)
    check(load().moe_prof_hbm_ceiling(int(nbytes), int(mode), ctypes.byref(g)), "moe_prof_hbm_ceiling")
    return float(g.value)


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return MOE_F32
    if dt == torch.bfloat16:
        return MOE_BF16
    raise TypeError(f"moe_mi355 supports float32 and bfloat16 tensors, got {dt}")


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one ROCm device; CPU tensors are rejected."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "moe_mi355 runs on an AMD Instinct GPU (gfx950) only; got a tensor on "
                f"{t.device}. Move the module and inputs to the GPU."
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"moe_mi355: tensors on different devices ({dev} vs {t.device})")
    return dev


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_ws_cache = {}
_ARENA_BYTES = 32 << 20
_capture_arena = {}  # device index -> [zeroed buffer, bytes handed out]


def workspace(nbytes: int, device: torch.device, key: Optional[str] = None) -> torch.Tensor:
    """Scratch memory for one call.  With ``key``, a workspace that must start zeroed and that the kernels
    leave zeroed where it matters (the router forward's ticket counter): one zero-initialised buffer per
    (key, device, stream), reused by every call on that stream (stream order serialises them).  Under
    graph capture each capture takes a fresh slice of a per-device arena zeroed (and synchronised) once
    outside any capture, so the graph holds no fill node (a zeroed buffer made inside the capture once the
    arena is used up)."""
    n = max(int(nbytes), 1)
    if key is None:
        return torch.empty(n, dtype=torch.uint8, device=device)
    arena = _capture_arena.get(device.index)
    if torch.cuda.is_current_stream_capturing():
        n256 = (n + 255) // 256 * 256
        if arena is not None and arena[1] + n256 <= _ARENA_BYTES:
            buf = arena[0].narrow(0, arena[1], n)
            arena[1] += n256
            return buf
        return torch.zeros(n, dtype=torch.uint8, device=device)
    if arena is None:
        _capture_arena[device.index] = [torch.zeros(_ARENA_BYTES, dtype=torch.uint8, device=device), 0]
        torch.cuda.current_stream(device).synchronize()  # once: later captures may replay on any stream
    stream = torch.cuda.current_stream(device).cuda_stream
    k = (key, device.index, stream)
    buf = _ws_cache.get(k)
    if buf is None or buf.numel() < n:
        buf = torch.zeros(n, dtype=torch.uint8, device=device)
        _ws_cache[k] = buf
    return buf
