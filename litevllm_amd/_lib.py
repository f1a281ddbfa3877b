"""ctypes binding of ``libawq_w4a16.so`` (the C ABI declared in ``include/awq_w4a16.h``).

The library is built in-tree by ``litevllm_amd.build`` (``hipcc --offload-arch=gfx950``).
Loading fails loudly when it is missing: there is no CPU or eager-PyTorch fallback.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libawq_w4a16.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

# constants mirrored from include/awq_w4a16.h
LAYOUT_AUTOAWQ = 0
LAYOUT_KN_SEQ = 1
LAYOUT_NK_SEQ = 2
LAYOUT_DECODE_STREAM = 3
LAYOUT_DECODE_NARROW = 4

DTYPE_NONE = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2
DTYPE_F32 = 3

OK = 0
ERR_NULL = 1
ERR_SHAPE = 2
ERR_UNSUPPORTED = 3
ERR_WORKSPACE = 4
ERR_LAUNCH = 5
ERR_STRIDE = 6

# name -> (restype, argtypes); every symbol include/awq_w4a16.h declares
_c_i32, _c_i64, _c_sz, _c_p = ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p
SIGNATURES = {
    "awq_w4a16_version": (ctypes.c_int, []),
    "awq_w4a16_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "awq_w4a16_dequant": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32,
                                         _c_i32, _c_i32, _c_p]),
    "awq_w4a16_gemm_workspace_bytes": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32]),
    "awq_w4a16_gemm": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64,
                                      _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                      _c_i32, _c_p, _c_sz, _c_p]),
    "awq_w4a16_repack_nk_to_autoawq": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64,
                                                      _c_i64, _c_i32, _c_p]),
    "awq_w4a16_decode_stream_bytes": (_c_i64, [_c_i64, _c_i64]),
    "awq_w4a16_decode_narrow_bytes": (_c_i64, [_c_i64, _c_i64]),
    "awq_w4a16_pack_decode_narrow": (ctypes.c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_p]),
    "awq_w4a16_pack_decode_stream": (ctypes.c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_p]),
    "awq_w4a16_moe_stream_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i32]),
    "awq_w4a16_moe_pack_stream": (ctypes.c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p]),
    "awq_w4a16_moe_route": (ctypes.c_int, [_c_p, _c_i64, _c_i32, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_p,
                                           _c_p]),
    "awq_w4a16_moe_route_ex": (ctypes.c_int, [_c_p, _c_i64, _c_i32, _c_i64, _c_i32, _c_i32, ctypes.c_uint32,
                                              _c_p, _c_i32, _c_p, _c_p]),
    "awq_w4a16_probe_read": (ctypes.c_int, [_c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_p]),
    "awq_w4a16_gemm_rows_exact_workspace_bytes": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32]),
    "awq_w4a16_gemm_rows_exact": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64,
                                                 _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                                 _c_i32, _c_p, _c_sz, _c_p]),
    "awq_w4a16_gemm_noalloc_max_workspace": (_c_sz, []),
    "awq_w4a16_gemm_noalloc": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64,
                                              _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_p]),
    "awq_w4a16_moe_workspace_bytes": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i32, _c_i32]),
    "awq_w4a16_moe": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_i32, _c_p, _c_i32, _c_p, _c_p, _c_p, _c_p, _c_p,
                                     _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32,
                                     _c_i32, _c_i32, _c_i32, _c_p, _c_sz, _c_p]),
    "awq_w4a16_gate_up_interleave": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_p]),
    "awq_w4a16_gate_up_workspace_bytes": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32]),
    "awq_w4a16_gate_up_act": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64,
                                             _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_p,
                                             _c_sz, _c_p]),
    "awq_w4a16_rmsnorm": (ctypes.c_int, [_c_p, _c_i64, _c_p, ctypes.c_float, _c_p, _c_i64, _c_i64, _c_i64,
                                         _c_i32, _c_i32, _c_p]),
    "awq_w4a16_rmsnorm_gemm_workspace_bytes": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32]),
    "awq_w4a16_rmsnorm_gemm": (ctypes.c_int, [_c_p, _c_i64, _c_p, ctypes.c_float, _c_p, _c_p, _c_p, _c_p,
                                              _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32,
                                              _c_i32, _c_i32, _c_p, _c_sz, _c_p]),
}

MOE_ACT_SILU = 0
MOE_ACT_GELU_TANH = 1

ROUTE_RENORMALIZE = 1
ROUTE_SOFTMAX_IN_LOGITS_DTYPE = 2
ROUTE_CLAMP_SUM = 4

_lock = threading.Lock()
_lib = None


class AWQKernelError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, fn: str, code: int):
        self.code = int(code)
        super().__init__(f"{fn} failed with code {code}: {strerror(code)}")


def load(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and return the library; raises ``OSError`` if it is not built."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.isfile(p):
            raise OSError(
                f"{LIB_NAME} not found at {p}: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
            )
        lib = ctypes.CDLL(p)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


_num_cus = None


def num_cus() -> int:
    """Compute units of the current device (256 on MI355X; 256 when no GPU is visible)."""
    global _num_cus
    if _num_cus is None:
        try:
            import torch
            _num_cus = int(torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count)
        except Exception:
            _num_cus = 256
    return _num_cus


def strerror(code: int) -> str:
    try:
        return load().awq_w4a16_strerror(int(code)).decode()
    except OSError:
        return f"error {code}"


def check(fn: str, code: int) -> None:
    if code != OK:
        raise AWQKernelError(fn, code)
