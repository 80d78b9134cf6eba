"""ctypes binding of ``liballoy_amd.so`` (the C ABI declared in ``include/alloy_amd.h``).

The library is loaded from ``alloy_amd/csrc/liballoy_amd.so``.  There is no
fallback: if it is missing, every entry point raises ``LibraryMissing`` (a
RuntimeError) naming the path and how to build it.
"""

from __future__ import annotations

import ctypes
import pathlib
import threading

LIB_PATH = pathlib.Path(__file__).resolve().parent / "csrc" / "liballoy_amd.so"

# status codes (alloy_status)
OK, E_SHAPE, E_DTYPE, E_ALIGN, E_UNSUPPORTED, E_HIP, E_ARG = range(7)
# formats (alloy_format)
FMT = {"q8_0": 0, "q5_0": 1, "q4_k": 2, "q6_k": 3, "mlx_q4": 4, "q8_0_split": 5, "q5_0_split": 6}
ACT = {"silu": 0, "gelu": 1}
# dtypes (alloy_dtype)
DT_F32, DT_F16 = 0, 1
# paths (alloy_path)
PATH = {"auto": 0, "gemv": 1, "gemv_mfma": 2, "gemm": 3}

_EXC = {
    E_SHAPE: ValueError,
    E_DTYPE: TypeError,
    E_ALIGN: ValueError,
    E_UNSUPPORTED: NotImplementedError,
    E_HIP: RuntimeError,
    E_ARG: ValueError,
}


class LibraryMissing(RuntimeError):
    pass


_vp, _i32, _i64, _sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/alloy_amd.h
SIGNATURES = {
    "alloy_qmm": (_i32, [_i32, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _i64, _i32, _i64, _vp]),
    "alloy_qmm_ws": (_i32, [_i32, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _i64, _i32, _i64, _vp,
                            _i64, _vp]),
    "alloy_gemm_workspace_bytes": (_i64, [_i32, _i64, _i64, _i64]),
    "alloy_gguf_q4_k_mm": (_i32, [_vp, _i32, _vp, _vp, _i32, _i64, _i64, _i64, _vp]),
    "alloy_gguf_q6_k_mm": (_i32, [_vp, _i32, _vp, _vp, _i32, _i64, _i64, _i64, _vp]),
    "alloy_gguf_q8_0_mm": (_i32, [_vp, _i32, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp]),
    "alloy_gguf_q5_0_mm": (_i32, [_vp, _i32, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp]),
    "alloy_gguf_q8_0_blocks_mm": (_i32, [_vp, _i32, _vp, _vp, _i32, _i64, _i64, _i64, _vp]),
    "alloy_gguf_q5_0_blocks_mm": (_i32, [_vp, _i32, _vp, _vp, _i32, _i64, _i64, _i64, _vp]),
    "alloy_mlx_q4_mm": (_i32, [_vp, _i32, _vp, _vp, _vp, _i32, _vp, _i32, _i64, _i64, _i64, _vp]),
    "alloy_dequant": (_i32, [_i32, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _i64, _i64, _i64, _i64, _vp]),
    "alloy_moe_router_topk": (_i32, [_vp, _vp, _vp, _i64, _i32, _i32, _vp]),
    "alloy_moe_workspace_bytes": (_sz, [_i64, _i32, _i32, _i64, _i64]),
    "alloy_mlx_moe_routed": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i64, _i64, _i64, _vp, _sz, _vp, _vp]),
    "alloy_gguf_moe_routed": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i64, _i64, _i64, _vp, _sz, _vp, _vp]),
    "alloy_gguf_moe_routed_noalloc": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i64, _i64, _i64, _vp, _vp]),
    "alloy_embedding": (_i32, [_i32, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _i64, _i64, _i64, _vp, _vp]),
    "alloy_qmm_batched": (_i32, [_i32, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _vp]),
    "alloy_glu_workspace_bytes": (_sz, [_i32, _i64, _i64, _i64, _i32, _i32]),
    "alloy_qmm_glu": (_i32, [_i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _i64, _vp, _sz, _vp]),
    "alloy_gguf_q4_k_silu": (_i32, [_vp, _i32, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp, _sz, _vp]),
    "alloy_gguf_q4_k_gelu": (_i32, [_vp, _i32, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp, _sz, _vp]),
    "alloy_mlx_q4_silu": (_i32, [_vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _i64, _i64, _i64, _vp, _sz, _vp]),
    "alloy_gguf_q8_0_silu": (_i32, [_vp, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _vp, _sz, _vp]),
    "alloy_last_error": (ctypes.c_char_p, []),
    "alloy_version": (ctypes.c_char_p, []),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library (raises LibraryMissing when it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise LibraryMissing(
                    f"{LIB_PATH} not found: build it with `make -C {LIB_PATH.parent}` "
                    "or `python -c 'import __graft_entry__ as g; g.build()'`"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def check(status: int) -> None:
    """Map an alloy_status to the reference's exception types."""
    if status == OK:
        return
    msg = lib().alloy_last_error().decode(errors="replace")
    raise _EXC.get(status, RuntimeError)(msg or f"alloy_amd status {status}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
