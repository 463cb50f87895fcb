"""ctypes binding of libnkilab_hip.so (the C ABI declared in include/nkilab_hip.h).

The library is loaded once, from this package directory.  There is no
fallback: if the library is missing or no ROCm GPU is visible, the ops raise.
"""
from __future__ import annotations

import ctypes
import os

LIB_NAME = "libnkilab_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

F32, BF16, F16 = 0, 1, 2
GEMM_BLOCKED, GEMM_NAIVE = 0, 1
ABI_VERSION = 1

_c_int, _c_long, _c_float, _c_size = ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_size_t
_vp = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/nkilab_hip.h one for one.
SIGNATURES = {
    "nkl_abi_version": (_c_int, []),
    "nkl_last_error_string": (ctypes.c_char_p, []),
    "nkl_gemm": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_long, _c_long, _c_long, _c_long,
                          _c_int, _c_int, _c_long, _c_long, _c_long, _c_long, _c_int, _c_int, _c_int, _vp]),
    "nkl_gemm_swiglu": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_long, _c_long, _c_long, _c_int, _vp]),
    "nkl_check_blocks": (_c_int, [_c_int, _c_int]),
    "nkl_softmax": (_c_int, [_vp, _vp, _c_int, _c_int, _c_long, _c_long, _c_int, _vp]),
    "nkl_softmax_unfused_workspace_bytes": (_c_size, [_c_int, _c_int]),
    "nkl_softmax_unfused": (_c_int, [_vp, _vp, _vp, _c_size, _c_int, _c_int, _c_long, _c_long, _c_int, _vp]),
    "nkl_rmsnorm": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_long, _c_long, _c_float, _c_int, _c_int, _vp]),
    "nkl_rmsnorm_ex": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_long, _c_long, _c_float, _c_int, _c_int, _c_int,
                                _vp]),
    "nkl_swiglu": (_c_int, [_vp, _vp, _vp, _c_long, _c_int, _vp]),
    "nkl_stream_copy": (_c_int, [_vp, _vp, _c_long, _vp]),
    "nkl_split_bf16": (_c_int, [_vp, _vp, _c_int, _c_int, _c_long, _c_long, _vp]),
    "nkl_flash_attn_causal": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_long, _c_long, _c_long,
                                       _c_long, _c_long, _c_long, _c_long, _c_long, _c_float, _c_int, _vp]),
    "nkl_flash_attn_causal_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "nkl_flash_attn_causal_counter_bytes": (_c_size, [_c_int, _c_int, _c_int]),
    "nkl_flash_attn_causal_ws": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_size, _vp, _c_size, _c_int, _c_int, _c_int,
                                          _c_long, _c_long, _c_long, _c_long, _c_long, _c_long, _c_long, _c_long,
                                          _c_float, _c_int, _vp]),
    "nkl_flash_attn_causal_gqa": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_size, _vp, _c_size, _c_int, _c_int, _c_int,
                                           _c_int, _c_long, _c_long, _c_long, _c_long, _c_long, _c_long, _c_long,
                                           _c_long, _c_float, _c_int, _vp]),
    "nkl_flash_attn_causal_noalloc": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_long,
                                               _c_long, _c_long, _c_long, _c_long, _c_long, _c_long, _c_long,
                                               _c_float, _c_int, _vp]),
    "nkl_attention_naive_gqa": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_size, _c_int, _c_int, _c_int, _c_int, _c_long,
                                         _c_long, _c_long, _c_long, _c_long, _c_long, _c_long, _c_long, _c_float,
                                         _c_int, _vp]),
    "nkl_rope": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _c_long, _c_long, _c_long, _c_long, _c_int, _c_float,
                          _c_int, _vp]),
    "nkl_flash_attn_configure": (_c_int, [_c_int, _c_int, _c_int, _c_int]),
    "nkl_flash_attn_configure_polls": (_c_int, [_c_int]),
    "nkl_flash_attn_plan_check": (_c_int, [_c_int, _c_int, _c_int, _c_int, _vp]),
    "nkl_attention_naive_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int]),
    "nkl_attention_naive": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_size, _c_int, _c_int, _c_int, _c_long, _c_long,
                                     _c_long, _c_long, _c_long, _c_long, _c_long, _c_long, _c_float, _c_int, _vp]),
}

_lib = None


class NklError(RuntimeError):
    """A negative status returned by the HIP library."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP kernel library."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m nkilab.build` (or __graft_entry__.build())")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, args
        ver = handle.nkl_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {ver}, expected {ABI_VERSION}; rebuild it")
        _lib = handle
    return _lib


# Codes of nkl_flash_attn_configure (include/nkilab_hip.h).
FLASH_KERNELS = {"teams": 0, "w1": 1, "w64": 2, "w64x4": 3, "teams4": 4, "w1o2": 5, "fwd": 6, "pp": 7, "ks": 8,
                 "tiny": 9}
FLASH_SCHEDULES = {"block": 0, "balanced": 1, "pairs": 2}


def flash_configure(kernel: str | None = None, schedule: str | None = None, qb: int | None = None,
                    cpb: int | None = None) -> None:
    """Force the bf16 attention kernel / schedule / block / block start cost
    (None: the automatic choice) for every later call in this process."""
    call("nkl_flash_attn_configure", FLASH_KERNELS[kernel] if kernel else -1,
         FLASH_SCHEDULES[schedule] if schedule else -1, int(qb) if qb else -1, -1 if cpb is None else int(cpb))


def flash_configure_polls(polls: int | None = None) -> None:
    """Set the poll budget of the workgroup that merges a split query block
    (None: the automatic choice; 0: never wait, the last part to arrive merges)."""
    call("nkl_flash_attn_configure_polls", -1 if polls is None else int(polls))


def flash_plan_check(H: int, S: int, d: int, f16: bool = False) -> tuple[int, int, int, int, int]:
    """Check on the host the work split the 16-bit attention kernels would
    walk for an H x S x d call under the configuration in force; raise
    NklError naming the first broken invariant.  Returns (workgroups, units,
    split blocks, most parts of one block, merge poll budget or -1 without
    the balanced schedule)."""
    info = (ctypes.c_long * 5)()
    call("nkl_flash_attn_plan_check", int(H), int(S), int(d), 2 if f16 else 1, info)
    return tuple(info)


def call(name: str, *args) -> int:
    """Call a status-returning entry point and raise on failure."""
    L = lib()
    rc = getattr(L, name)(*args)
    if rc != 0:
        msg = L.nkl_last_error_string().decode(errors="replace")
        if rc == -1 and "PSUM" not in msg:
            raise ValueError(f"{name}: {msg}")
        raise NklError(name, rc, msg)
    return rc
