"""Torch-facing wrappers of the C ABI: device memory and streams come from PyTorch,
every byte of arithmetic runs in the HIP kernels of ``libawq_w4a16.so``.

Layouts (``layout=`` keyword everywhere):
  * ``"ref"``      reference runtime layout: qweight int32 [N, K/8] (sequential nibbles),
                   scales [N, K/G], qzeros int32 [N, ceil(K/G/8)]
  * ``"autoawq"``  AutoAWQ layout: qweight int32 [K, N/8] (order 0,2,4,6,1,3,5,7),
                   scales [K/G, N], qzeros int32 [K/G, N/8]
  * ``"kn_seq"``   [K, N/8] with sequential nibbles (the reference dequant's row-grouped geometry)

Decode-shaped calls (M <= 32, fp16 activations and scales, group 32/64/128) read a one-time,
lossless re-ordering of the AutoAWQ qweight (the library's decode stream layout) that the
decode kernel streams as contiguous 8 KiB runs.  It is built on first use and cached per
weight tensor, the way the reference caches derived packs on its weight objects
(``tensor.py:1251-1256``); ``prepare_decode_stream`` builds it ahead of time.
"""
from __future__ import annotations

import threading
import weakref

import torch

from . import _lib as L

LAYOUTS = {"autoawq": L.LAYOUT_AUTOAWQ, "kn_seq": L.LAYOUT_KN_SEQ, "ref": L.LAYOUT_NK_SEQ}
_DT = {torch.float16: L.DTYPE_F16, torch.bfloat16: L.DTYPE_BF16, torch.float32: L.DTYPE_F32}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DT[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}") from None


def layout_code(layout: str) -> int:
    try:
        return LAYOUTS[layout]
    except KeyError:
        raise ValueError(f"unknown layout {layout!r}; expected one of {sorted(LAYOUTS)}") from None


def _stream_ptr(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else int(t.data_ptr())


def _require_device(*tensors: torch.Tensor | None) -> torch.device:
    """All tensors on one GPU; the kernels dereference these pointers on the device."""
    devs = {t.device for t in tensors if t is not None}
    if len(devs) != 1:
        raise ValueError(f"tensors must share one device, got {sorted(map(str, devs))}")
    dev = devs.pop()
    if dev.type != "cuda":
        raise ValueError(f"HIP kernels need GPU tensors, got device {dev}")
    return dev


def gemm_dims(qweight: torch.Tensor, layout: str) -> tuple[int, int]:
    """(K, N) of a packed weight in the given layout."""
    if layout == "ref":
        return int(qweight.shape[1]) * 8, int(qweight.shape[0])
    return int(qweight.shape[0]), int(qweight.shape[1]) * 8


# ------------------------------------------------------------------ dequant
def dequant(qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor | None,
            group_size: int, layout: str = "ref", out_dtype: torch.dtype = torch.float16,
            out: torch.Tensor | None = None) -> torch.Tensor:
    """Unpacked matrix in the packed tensor's orientation: ``ref`` -> [N, K], else [K, N]."""
    lib = L.load()
    _require_device(qweight, scales, qzeros, out)
    rows = int(qweight.shape[0])
    cols = int(qweight.shape[1]) * 8
    if out is None:
        out = torch.empty((rows, cols), dtype=out_dtype, device=qweight.device)
    qweight, scales = qweight.contiguous(), scales.contiguous()
    qzeros = qzeros.contiguous() if qzeros is not None else None
    rc = lib.awq_w4a16_dequant(_ptr(qweight), _ptr(scales), _ptr(qzeros), _ptr(out), rows, cols,
                               int(group_size), layout_code(layout), dtype_code(scales.dtype),
                               dtype_code(out.dtype), _stream_ptr(qweight.device))
    L.check("awq_w4a16_dequant", rc)
    return out


# ------------------------------------------------------------------ repack
def repack_ref_to_autoawq(qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor | None,
                          group_size: int):
    """Reference layout -> AutoAWQ layout on the device (lossless)."""
    lib = L.load()
    _require_device(qweight, scales, qzeros)
    n, k = int(qweight.shape[0]), int(qweight.shape[1]) * 8
    ng = k // int(group_size)
    dev = qweight.device
    qw = torch.empty((k, n // 8), dtype=torch.int32, device=dev)
    sc = torch.empty((ng, n), dtype=scales.dtype, device=dev)
    qz = torch.empty((ng, n // 8), dtype=torch.int32, device=dev) if qzeros is not None else None
    qweight, scales = qweight.contiguous(), scales.contiguous()
    qzeros = qzeros.contiguous() if qzeros is not None else None
    rc = lib.awq_w4a16_repack_nk_to_autoawq(_ptr(qweight), _ptr(qzeros), _ptr(scales), _ptr(qw),
                                            _ptr(qz), _ptr(sc), n, k, int(group_size),
                                            _stream_ptr(dev))
    L.check("awq_w4a16_repack_nk_to_autoawq", rc)
    return qw, sc, qz


def pack_decode_stream(qweight: torch.Tensor) -> torch.Tensor:
    """AutoAWQ (or kn_seq) qweight [K, N/8] -> the decode stream layout (int32, flat)."""
    lib = L.load()
    _require_device(qweight)
    if qweight.dtype != torch.int32 or qweight.dim() != 2:
        raise ValueError("qweight must be a 2-D int32 tensor [K, N/8]")
    k, n = int(qweight.shape[0]), int(qweight.shape[1]) * 8
    nbytes = int(lib.awq_w4a16_decode_stream_bytes(k, n))
    if nbytes <= 0:
        raise ValueError(f"no decode stream layout for K={k}, N={n} (need K % 32 == 0)")
    qweight = qweight.contiguous()
    out = torch.empty(nbytes // 4, dtype=torch.int32, device=qweight.device)
    rc = lib.awq_w4a16_pack_decode_stream(_ptr(qweight), _ptr(out), k, n, _stream_ptr(qweight.device))
    L.check("awq_w4a16_pack_decode_stream", rc)
    return out


class _DerivedCache:
    """Caches tensors derived from a packed weight, keyed by the source tensors' storage
    pointers, shapes and version counters and checked against a weak reference to the
    source (the role the reference's derived-pack cache plays at tensor.py:1251-1256)."""

    def __init__(self, build, capacity: int = 1024):
        self.build = build
        self.capacity = capacity
        self._d: dict = {}
        self._lock = threading.Lock()

    @staticmethod
    def _key(*tensors):
        return tuple(None if t is None else (t.data_ptr(), tuple(t.shape), t._version, t.device.index)
                     for t in tensors)

    def get(self, src: torch.Tensor, *others, args=()):
        key = (self._key(src, *others), args)
        with self._lock:
            hit = self._d.get(key)
            if hit is not None:
                ref, val = hit
                if ref() is src:
                    return val
        val = self.build(src, *others, *args)
        with self._lock:
            # drop entries whose source tensor is gone, then the oldest beyond capacity
            for k in [k for k, (r, _) in self._d.items() if r() is None]:
                del self._d[k]
            while len(self._d) >= self.capacity:
                self._d.pop(next(iter(self._d)))
            self._d[key] = (weakref.ref(src), val)
        return val

    def clear(self):
        with self._lock:
            self._d.clear()


def _repack_builder(qweight, scales, qzeros, group_size):
    return repack_ref_to_autoawq(qweight, scales, qzeros, group_size)


REPACK_CACHE = _DerivedCache(_repack_builder)
STREAM_CACHE = _DerivedCache(pack_decode_stream)


def prepare_decode_stream(qweight: torch.Tensor) -> torch.Tensor:
    """Build (and cache) the decode stream copy of an AutoAWQ qweight ahead of the first call."""
    return STREAM_CACHE.get(qweight)


# ------------------------------------------------------------------ workspace
class _Workspace:
    """Zero-initialised split-K scratch, one per device.  The kernels leave its counter
    region at zero, so a buffer is zeroed only when it is (re)allocated.  Calls are
    serialised on the caller's stream (the reference issues every AWQ matmul from one
    engine thread on the current stream); work on two streams at once needs
    ``reserve(device, nbytes, key)`` with distinct keys."""

    def __init__(self):
        self._bufs: dict = {}
        self._lock = threading.Lock()

    def get(self, device: torch.device, nbytes: int, key=None) -> torch.Tensor:
        k = (device.index, key)
        with self._lock:
            buf = self._bufs.get(k)
            if buf is None or buf.numel() < nbytes:
                size = max(nbytes, 16 << 20)
                buf = torch.zeros(size, dtype=torch.uint8, device=device)
                self._bufs[k] = buf
            return buf

    reserve = get


WORKSPACE = _Workspace()


# ------------------------------------------------------------------ GEMM
DECODE_MAX_M = 32
# packed words per lane of the library's decode stream layout (decode_stream_wpl in csrc)
DECODE_STREAM_WPL = 1
DECODE_GROUPS = (32, 64, 128)


def _use_decode_stream(M, K, group_size, a, scales, layout, decode_stream):
    if decode_stream is False or layout != "autoawq":
        return False
    eligible = (M <= DECODE_MAX_M and int(group_size) in DECODE_GROUPS and K % 32 == 0
                and a.dtype == torch.float16 and scales.dtype == torch.float16)
    if decode_stream is True and not eligible:
        raise ValueError("the decode stream layout needs M <= 32, group 32/64/128 and fp16 "
                         "activations and scales")
    return eligible


def gemm(a: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor | None,
         group_size: int, bias: torch.Tensor | None = None, split_k: int = 0,
         layout: str = "ref", out: torch.Tensor | None = None,
         decode_stream: bool | None = None) -> torch.Tensor:
    """``out[M, N] = a[M, K] @ dequant(W)^T (+ bias)`` on the HIP kernels.

    ``split_k = 0`` lets the library choose its K partition; any value >= 1 fixes it
    (results are bitwise reproducible for a fixed value).  ``decode_stream`` (default: when
    eligible) routes decode-shaped calls through the cached decode stream copy of the weight.
    """
    lib = L.load()
    if a.dim() != 2:
        raise ValueError("a must be 2-D")
    _require_device(a, qweight, scales, qzeros, bias, out)
    K, N = gemm_dims(qweight, layout)
    M = int(a.shape[0])
    if int(a.shape[1]) != K:
        raise ValueError(f"K mismatch: a has {a.shape[1]}, weight has {K}")
    if layout == "ref":
        qweight, scales, qzeros = REPACK_CACHE.get(qweight, scales, qzeros, args=(int(group_size),))
        layout = "autoawq"
    a = a.contiguous()
    qweight, scales = qweight.contiguous(), scales.contiguous()
    qzeros = qzeros.contiguous() if qzeros is not None else None
    if out is None:
        out = torch.empty((M, N), dtype=a.dtype, device=a.device)
    if bias is not None:
        bias = bias.contiguous()
    dev = a.device
    stream = _stream_ptr(dev)
    lc = layout_code(layout)
    if _use_decode_stream(M, K, group_size, a, scales, layout, decode_stream):
        qweight = STREAM_CACHE.get(qweight)
        lc = L.LAYOUT_DECODE_STREAM
    ws_bytes = int(lib.awq_w4a16_gemm_workspace_bytes(M, N, K, int(group_size), int(split_k), lc))
    ws = WORKSPACE.get(dev, ws_bytes) if ws_bytes else None
    rc = lib.awq_w4a16_gemm(
        _ptr(a), int(a.stride(0)), _ptr(qweight), _ptr(scales), _ptr(qzeros), _ptr(bias), _ptr(out),
        int(out.stride(0)), M, N, K, int(group_size), int(split_k), lc, dtype_code(a.dtype),
        dtype_code(scales.dtype), dtype_code(bias.dtype) if bias is not None else L.DTYPE_NONE,
        _ptr(ws), ws_bytes if ws is not None else 0, stream)
    L.check("awq_w4a16_gemm", rc)
    return out
