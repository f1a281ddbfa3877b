"""Torch-facing wrappers of the C ABI: device memory and streams come from PyTorch,
every byte of arithmetic runs in the HIP kernels of ``libawq_w4a16.so``.

Layouts (``layout=`` keyword everywhere):
  * ``"ref"``      reference runtime layout: qweight int32 [N, K/8] (sequential nibbles),
                   scales [N, K/G], qzeros int32 [N, ceil(K/G/8)]
  * ``"autoawq"``  AutoAWQ layout: qweight int32 [K, N/8] (order 0,2,4,6,1,3,5,7),
                   scales [K/G, N], qzeros int32 [K/G, N/8]
  * ``"kn_seq"``   [K, N/8] with sequential nibbles (the reference dequant's row-grouped geometry)

Calls read a one-time, lossless re-ordering of the packed qweight that their kernel streams
contiguously (the narrow or the stream decode layout; prefill reads the stream layout).  It is
built on first use and held by the weight tensor itself, the way the reference holds derived
packs on its weight objects (``tensor.py:1251-1256``); ``prepare_decode_stream`` builds it ahead
of time and ``derived_copies`` lists what a weight holds.
"""
from __future__ import annotations

import threading

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


def pack_decode_narrow(qweight: torch.Tensor) -> torch.Tensor:
    """AutoAWQ qweight [K, N/8] -> the narrow decode layout (int32, flat)."""
    lib = L.load()
    _require_device(qweight)
    if qweight.dtype != torch.int32 or qweight.dim() != 2:
        raise ValueError("qweight must be a 2-D int32 tensor [K, N/8]")
    k, n = int(qweight.shape[0]), int(qweight.shape[1]) * 8
    nbytes = int(lib.awq_w4a16_decode_narrow_bytes(k, n))
    if nbytes <= 0:
        raise ValueError(f"no narrow decode layout for K={k}, N={n} (need K % 32 == 0)")
    qweight = qweight.contiguous()
    out = torch.empty(nbytes // 4, dtype=torch.int32, device=qweight.device)
    rc = lib.awq_w4a16_pack_decode_narrow(_ptr(qweight), _ptr(out), k, n, _stream_ptr(qweight.device))
    L.check("awq_w4a16_pack_decode_narrow", rc)
    return out


_DERIVED_ATTR = "_awq_derived"
_DERIVED_LOCK = threading.Lock()


class _DerivedCache:
    """Tensors derived from a packed weight (a repack, a kernel-layout copy, a concatenation),
    held by the source tensor object itself, as the reference holds its derived packs on the
    weight object (``tensor.py:1251-1256``): they live exactly as long as the weight, and no
    module-global table grows, evicts or rebuilds them.  An entry is reused while the source
    and the other inputs are the same storage, shape and version (an in-place update of any of
    them rebuilds it); one entry per cache and source tensor."""

    def __init__(self, name: str, build):
        self.name = name
        self.build = build

    @staticmethod
    def _key(*tensors):
        return tuple(None if t is None else (t.data_ptr(), tuple(t.shape), t._version, t.device.index)
                     for t in tensors)

    def get(self, src: torch.Tensor, *others, args=()):
        key = (self._key(src, *others), args)
        store = src.__dict__.get(_DERIVED_ATTR)
        hit = store.get(self.name) if store is not None else None
        if hit is not None and hit[0] == key:
            return hit[1]
        val = self.build(src, *others, *args)
        with _DERIVED_LOCK:
            store = src.__dict__.setdefault(_DERIVED_ATTR, {})
            store[self.name] = (key, val)
        return val

    def held(self, src: torch.Tensor):
        """The value this cache holds on ``src`` (whatever its key), or None."""
        hit = (src.__dict__.get(_DERIVED_ATTR) or {}).get(self.name)
        return None if hit is None else hit[1]


def derived_copies(src: torch.Tensor) -> dict:
    """Name -> value of every derived pack a weight tensor holds (for inspection and tests)."""
    return {k: v[1] for k, v in (src.__dict__.get(_DERIVED_ATTR) or {}).items()}


def _repack_sz_builder(qweight, scales, qzeros, group_size):
    """Scales and zeros of a reference-layout weight in the AutoAWQ layout the kernels read
    (about 4 % of the weight's bytes); the repacked qweight is not kept."""
    _, sc, qz = repack_ref_to_autoawq(qweight, scales, qzeros, group_size)
    return sc, qz


def _repack_qw_builder(qweight, scales, qzeros, group_size):
    return repack_ref_to_autoawq(qweight, scales, qzeros, group_size)[0]


def _ref_stream_builder(qweight, scales, qzeros, group_size):
    return pack_decode_stream(repack_ref_to_autoawq(qweight, scales, qzeros, group_size)[0])


def _ref_narrow_builder(qweight, scales, qzeros, group_size):
    return pack_decode_narrow(repack_ref_to_autoawq(qweight, scales, qzeros, group_size)[0])


# AutoAWQ-layout weights: the kernel copies are built from the tensor itself
STREAM_CACHE = _DerivedCache("decode_stream", pack_decode_stream)
NARROW_CACHE = _DerivedCache("decode_narrow", pack_decode_narrow)
# reference-layout weights: repacked scales and zeros, and kernel copies built through a
# transient AutoAWQ repack; the AutoAWQ qweight is kept only for the kernels that read it
REF_SZ_CACHE = _DerivedCache("ref_scales_zeros", _repack_sz_builder)
REF_QW_CACHE = _DerivedCache("ref_autoawq_qweight", _repack_qw_builder)
REF_STREAM_CACHE = _DerivedCache("ref_decode_stream", _ref_stream_builder)
REF_NARROW_CACHE = _DerivedCache("ref_decode_narrow", _ref_narrow_builder)


def prepare_decode_stream(qweight: torch.Tensor) -> torch.Tensor:
    """Build (and hold on the tensor) the decode stream copy of an AutoAWQ qweight ahead of the
    first call."""
    return STREAM_CACHE.get(qweight)


# ------------------------------------------------------------------ workspace
class _Workspace:
    """Zero-initialised split-K scratch, one per device.  The kernels leave its counter
    region at zero, so a buffer is zeroed only when it is (re)allocated.  Calls are
    serialised on the caller's stream (the reference issues every AWQ matmul from one
    engine thread on the current stream); work on two streams at once needs
    ``reserve(device, nbytes, key)`` with distinct keys.

    A buffer that has been handed out is never freed: when a larger one is needed, the old
    one stays alive (``_retired``), because HIP graphs captured earlier hold its address and
    write their counters and partials into it on every replay.  Sizes are powers of two (at
    least 16 MiB), so the retired buffers never add up to more than the live one.  ``reserve``
    the largest size up front to avoid regrowth altogether."""

    def __init__(self):
        self._bufs: dict = {}
        self._retired: list = []
        self._lock = threading.Lock()

    def get(self, device: torch.device, nbytes: int, key=None) -> torch.Tensor:
        k = (device.index, key)
        with self._lock:
            buf = self._bufs.get(k)
            if buf is None or buf.numel() < nbytes:
                if buf is not None:
                    self._retired.append(buf)
                # powers of two: the retired buffers of a growing size sum to less than the
                # live one, however small the steps of growth
                size = 1 << max(int(nbytes) - 1, (16 << 20) - 1).bit_length()
                buf = torch.zeros(size, dtype=torch.uint8, device=device)
                self._bufs[k] = buf
            return buf

    reserve = get


WORKSPACE = _Workspace()


# ------------------------------------------------------------------ GEMM
def out_problem(out: torch.Tensor, M: int, N: int, a: torch.Tensor) -> str | None:
    """Why a caller-supplied ``out`` cannot take an ``[M, N]`` result of ``a``'s dtype (the
    kernels write M x N 16-bit values at row stride ``out.stride(0)``), or None."""
    if tuple(out.shape) != (M, N):
        return "bad_output_shape"
    if out.dtype != a.dtype or out.device != a.device:
        return "bad_output"
    if N > 0 and M > 0 and (out.stride(1) != 1 or (M > 1 and out.stride(0) < N)):
        return "bad_output"
    return None


def check_out(out: torch.Tensor, M: int, N: int, a: torch.Tensor) -> None:
    """Raise ``ValueError`` before any launch when ``out`` cannot take the result."""
    why = out_problem(out, M, N, a)
    if why is not None:
        raise ValueError(f"{why}: out must be [{M}, {N}] {a.dtype} on {a.device} with unit column "
                         f"stride, got {tuple(out.shape)} {out.dtype} on {out.device}, strides {out.stride()}")


DECODE_MAX_M = 32
DECODE_GROUPS = (32, 64, 128)


def _decode_shaped(M, group_size):
    return M <= DECODE_MAX_M and int(group_size) in DECODE_GROUPS


def _use_decode_stream(M, K, N, group_size, layout, decode_stream):
    """Whether the call reads the stream copy of an AutoAWQ weight: the decode kernel's layout
    for decode shapes, and the layout of the prefill kernel that reads it (K % 32 == 0,
    power-of-two group size), which beats the AutoAWQ-layout prefill kernel at configs[3]'s
    shapes (measured on MI355X: M = 2048, K = 4096, N = 24576 369 against 395 us; N = 12288
    214 against 216 us; M = 512 136 against 146 us).  ``decode_stream=False`` keeps the
    AutoAWQ tensor."""
    if decode_stream is False or layout != "autoawq":
        return False
    g = int(group_size)
    if _decode_shaped(M, g):
        eligible = K % 32 == 0
    else:
        eligible = K % 32 == 0 and g & (g - 1) == 0
    if decode_stream is True and not eligible:
        raise ValueError("the stream layout needs K % 32 == 0 (and a power-of-two group size for M > 32)")
    return eligible


def _auto_splits(M: int, N: int, K: int) -> int:
    """The K partition count the library's planner picks for the 128-column stream kernel when
    split_k is 0 (``plan_decode``: about 32 k-steps per range, at most one round of blocks on
    the chip, at most one range per 64-row block)."""
    tiles = -(-N // 128)
    fit = max(1, L.num_cus() // tiles)
    by_k = max(1, (K // 32 + 16) // 32)
    return max(1, min(-(-K // 64), by_k, fit))


def _narrow_fits(M: int, N: int, K: int, split_k: int, bf16: bool = False) -> bool:
    """Whether a decode-shaped call reads the narrow layout (one block per 16 columns over the
    whole K, no split-K hand-off) instead of the 128-column stream.

    ``split_k = 0`` ("auto"): where the narrow kernel is faster (measured on MI355X: while the
    activation rows fit the kernel's LDS staging, M = 1 .. 4, up to four 16-column tiles per CU
    at M <= 3 and K <= 4096 (K = 4096, N = 11008 .. 16384: 7.7-10.7 us against 9.2-12.0 us for
    the stream kernel; at N = 20480 the stream kernel is ahead), up to three at K <= 8192
    (M = 4, N = 12288: 8.9 against 10.5 us; M = 1, K = 8192, N = 12288: 13.4 against 13.6 us),
    else up to two; with K <= 4096, up to three tiles per CU at M = 5 (N = 12288: 9.5 against
    10.7 us) and two at M = 6 .. 8 (K = 4096, N = 6144 / 8192: 7.6-8.6 us against 8.5-9.5 us
    for the stream kernel); otherwise one tile per CU with K <= 14336 up to M = 4, K <= 8192 up
    to M = 8 and K <= 4096 up to M = 16 (N = 4096: M = 4, K = 8192 7.9 against 9.2 us, K = 14336
    10.9 against 11.6 us; M = 8, K = 8192 8.9 against 9.4 us; M = 8, K = 14336 and every N = 6144
    case past those limits ran faster on the split stream kernel)).
    ``split_k = 1`` (the whole K per block, the reference's non-split kernel): the same kernel
    as auto wherever auto does not split K, so a forced 1 and auto give the same bits there;
    where auto would split, the narrow kernel, whose N / 16 blocks cover the chip that the
    N / 128 whole-K stream blocks leave mostly idle.
    ``split_k > 1`` fixes a partition of K, which only the stream kernel takes.
    ``bf16`` activations take the narrow kernel only at K <= 4096 with one tile per CU up to
    M = 16, or two at M = 1 (K = 4096, N = 4096: 6.1 / 6.5 / 7.9 us at M = 1 / 4 / 16 against
    7.6 / 7.8 / 9.2 us on the stream kernel; M = 1, N = 8192 8.9 against 9.4 us): their narrow
    path trails the stream kernel past that (M = 4, N = 6144 / 8192 9.9 / 10.2 against 8.5 /
    9.2 us; M = 1, K = 12288, N = 4096 12.5 against 10.6 us; M = 1, N = 12288 11.1 against
    9.5 us)."""
    if split_k > 1:
        return False
    tiles = -(-N // 16)
    if bf16:
        auto = K <= 4096 and ((M <= 16 and tiles <= L.num_cus()) or (M == 1 and tiles <= 2 * L.num_cus()))
        if split_k == 0 or auto:
            return auto
        return _auto_splits(M, N, K) > 1
    if M <= 4 and M * K * 2 <= 49152:
        per_cu = 4 if (M <= 3 and K <= 4096) else (3 if K <= 8192 else 2)
        auto = tiles <= per_cu * L.num_cus()
    elif M <= 8 and K <= 4096:
        auto = tiles <= (3 if M <= 5 else 2) * L.num_cus()
    else:
        auto = tiles <= L.num_cus() and ((M <= 4 and K <= 14336) or (M <= 8 and K <= 8192) or (M <= 16 and K <= 4096))
    if split_k == 0 or auto:
        return auto
    return _auto_splits(M, N, K) > 1


def _kernel_weight(qweight, scales, qzeros, group_size, layout, M, N, K, split_k, decode_stream, decode_layout,
                   bf16=False):
    """The weight copy and layout code the kernels read for this call.  Decode-shaped calls
    take the narrow or stream copy and prefill-sized ones the stream copy (see ``gemm``); both
    are held by the caller's weight tensor.  A reference-layout weight holds its scales and
    zeros in the AutoAWQ layout and the kernel copies built through a transient AutoAWQ repack;
    the repacked qweight itself is kept only when a kernel reads that layout directly
    (``decode_stream=False``, or a shape the stream layout does not cover)."""
    if decode_layout not in (None, "narrow", "stream"):
        raise ValueError(f"unknown decode_layout {decode_layout!r}")
    g = int(group_size)
    ref = layout == "ref"
    src_qw, src_sc, src_qz = qweight, scales, qzeros
    if ref:
        scales, qzeros = REF_SZ_CACHE.get(src_qw, src_sc, src_qz, args=(g,))
    else:
        scales = scales.contiguous()
        qzeros = qzeros.contiguous() if qzeros is not None else None
    if _use_decode_stream(M, K, N, g, "autoawq" if ref else layout, decode_stream):
        if decode_layout == "narrow" and not _decode_shaped(M, g):
            raise ValueError("the narrow layout needs M <= 32 and group 32/64/128")
        narrow = _decode_shaped(M, g) and (
            decode_layout == "narrow" or (decode_layout is None and _narrow_fits(M, N, K, int(split_k), bf16)))
        if ref:
            cache = REF_NARROW_CACHE if narrow else REF_STREAM_CACHE
            qweight = cache.get(src_qw, src_sc, src_qz, args=(g,))
        else:
            qweight = (NARROW_CACHE if narrow else STREAM_CACHE).get(qweight.contiguous())
        return qweight, scales, qzeros, (L.LAYOUT_DECODE_NARROW if narrow else L.LAYOUT_DECODE_STREAM)
    if ref:
        return REF_QW_CACHE.get(src_qw, src_sc, src_qz, args=(g,)), scales, qzeros, L.LAYOUT_AUTOAWQ
    return qweight.contiguous(), scales, qzeros, layout_code(layout)


def gemm(a: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor | None,
         group_size: int, bias: torch.Tensor | None = None, split_k: int = 0,
         layout: str = "ref", out: torch.Tensor | None = None,
         decode_stream: bool | None = None, decode_layout: str | None = None) -> torch.Tensor:
    """``out[M, N] = a[M, K] @ dequant(W)^T (+ bias)`` on the HIP kernels.

    ``split_k = 0`` lets the library choose its K partition; any value >= 1 fixes it
    (results are bitwise reproducible for a fixed value).  ``decode_stream`` (default: when
    eligible) routes decode-shaped calls through a cached derived copy of the weight:
    ``decode_layout`` "narrow" (16-column tiles, whole K per block), "stream" (128-column
    tiles, split-K) or None (narrow when N is small against the chip and split_k is 0).
    """
    lib = L.load()
    if a.dim() != 2:
        raise ValueError("a must be 2-D")
    _require_device(a, qweight, scales, qzeros, bias, out)
    K, N = gemm_dims(qweight, layout)
    M = int(a.shape[0])
    if int(a.shape[1]) != K:
        raise ValueError(f"K mismatch: a has {a.shape[1]}, weight has {K}")
    qweight, scales, qzeros, lc = _kernel_weight(qweight, scales, qzeros, group_size, layout, M, N, K,
                                                 split_k, decode_stream, decode_layout,
                                                 a.dtype == torch.bfloat16)
    # rows at any stride the kernels take (16-byte aligned, a multiple of 8 elements) are read in
    # place, as the reference's kernel takes stride_am; anything else is made contiguous
    lda = int(a.stride(0)) if M > 1 else K
    if a.stride(1) != 1 or lda < K or lda % 8 != 0 or a.data_ptr() % 16 != 0:
        a = a.contiguous()
        lda = K
    if out is None:
        out = torch.empty((M, N), dtype=a.dtype, device=a.device)
    else:
        check_out(out, M, N, a)
    if bias is not None:
        bias = bias.contiguous()
    dev = a.device
    stream = _stream_ptr(dev)
    ws_bytes = int(lib.awq_w4a16_gemm_workspace_bytes(M, N, K, int(group_size), int(split_k), lc))
    ws = WORKSPACE.get(dev, ws_bytes) if ws_bytes else None
    rc = lib.awq_w4a16_gemm(
        _ptr(a), lda, _ptr(qweight), _ptr(scales), _ptr(qzeros), _ptr(bias), _ptr(out),
        int(out.stride(0)), M, N, K, int(group_size), int(split_k), lc, dtype_code(a.dtype),
        dtype_code(scales.dtype), dtype_code(bias.dtype) if bias is not None else L.DTYPE_NONE,
        _ptr(ws), ws_bytes if ws is not None else 0, stream)
    L.check("awq_w4a16_gemm", rc)
    return out


def gemm_rows_exact(a: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor | None,
                    group_size: int, bias: torch.Tensor | None = None, split_k: int = 0, layout: str = "ref",
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """``gemm`` with every row computed exactly as a lone ``M = 1`` call computes it (the same
    weight copy, plan, kernel and reduction order), so ``out[m]`` equals ``gemm(a[m:m+1], ...)``
    bit for bit whatever the batch -- the contract of the reference's row-exact small-batch
    kernel (``awq_fused_gemm.py:1066-1143``).  One launch whose grid has a row of the M = 1
    call's blocks per input row (group sizes 32 / 64 / 128), as the reference's grid
    ``(cdiv(N, BN), M)``."""
    lib = L.load()
    if a.dim() != 2:
        raise ValueError("a must be 2-D")
    _require_device(a, qweight, scales, qzeros, bias, out)
    K, N = gemm_dims(qweight, layout)
    M = int(a.shape[0])
    if int(a.shape[1]) != K:
        raise ValueError(f"K mismatch: a has {a.shape[1]}, weight has {K}")
    # the weight copy and plan of an M = 1 call
    qweight, scales, qzeros, lc = _kernel_weight(qweight, scales, qzeros, group_size, layout, 1, N, K,
                                                 split_k, None, None, a.dtype == torch.bfloat16)
    a = a.contiguous()
    if out is None:
        out = torch.empty((M, N), dtype=a.dtype, device=a.device)
    else:
        check_out(out, M, N, a)
    if bias is not None:
        bias = bias.contiguous()
    dev = a.device
    ws_bytes = int(lib.awq_w4a16_gemm_rows_exact_workspace_bytes(M, N, K, int(group_size), int(split_k), lc))
    ws = WORKSPACE.get(dev, ws_bytes) if ws_bytes else None
    rc = lib.awq_w4a16_gemm_rows_exact(
        _ptr(a), int(a.stride(0)), _ptr(qweight), _ptr(scales), _ptr(qzeros), _ptr(bias), _ptr(out),
        int(out.stride(0)), M, N, K, int(group_size), int(split_k), lc, dtype_code(a.dtype),
        dtype_code(scales.dtype), dtype_code(bias.dtype) if bias is not None else L.DTYPE_NONE,
        _ptr(ws), ws_bytes if ws is not None else 0, _stream_ptr(dev))
    L.check("awq_w4a16_gemm_rows_exact", rc)
    return out


# ------------------------------------------------------------------ RMSNorm prologue
def rmsnorm(x: torch.Tensor, norm_w: torch.Tensor, eps: float = 1e-6, out: torch.Tensor | None = None) -> torch.Tensor:
    """The normalised rows ``fp16((x * rsqrt(mean(x^2) + eps)) * norm_w)`` the fused RMSNorm +
    GEMM feeds its GEMM (fp32 arithmetic, one rounding; fp16 whatever ``x``'s dtype)."""
    lib = L.load()
    if x.dim() != 2 or norm_w.dim() != 1 or int(norm_w.shape[0]) != int(x.shape[1]):
        raise ValueError("x must be [M, K] and norm_w [K]")
    dev = _require_device(x, norm_w, out)
    M, K = int(x.shape[0]), int(x.shape[1])
    x, norm_w = x.contiguous(), norm_w.contiguous()
    if out is None:
        out = torch.empty((M, K), dtype=torch.float16, device=dev)
    rc = lib.awq_w4a16_rmsnorm(_ptr(x), K, _ptr(norm_w), float(eps), _ptr(out), int(out.stride(0)), M, K,
                               dtype_code(x.dtype), dtype_code(norm_w.dtype), _stream_ptr(dev))
    L.check("awq_w4a16_rmsnorm", rc)
    return out


def rmsnorm_gemm(x: torch.Tensor, norm_w: torch.Tensor, eps: float, qweight: torch.Tensor,
                 scales: torch.Tensor, qzeros: torch.Tensor | None, group_size: int, layout: str = "ref",
                 split_k: int = 0, out: torch.Tensor | None = None, decode_stream: bool | None = None,
                 decode_layout: str | None = None) -> torch.Tensor:
    """``out[M, N] = rmsnorm(x, norm_w, eps) @ dequant(W)^T`` through ``awq_w4a16_rmsnorm_gemm``:
    the normalised fp16 rows, the GEMM on them (same kernels and weight copies as ``gemm``),
    the fp16 result, converted to bf16 for bf16 ``x``."""
    lib = L.load()
    if x.dim() != 2 or norm_w.dim() != 1:
        raise ValueError("x must be [M, K] and norm_w [K]")
    dev = _require_device(x, norm_w, qweight, scales, qzeros, out)
    K, N = gemm_dims(qweight, layout)
    M = int(x.shape[0])
    if int(x.shape[1]) != K or int(norm_w.shape[0]) != K:
        raise ValueError(f"K mismatch: x has {x.shape[1]}, norm_w {norm_w.shape[0]}, weight {K}")
    qweight, scales, qzeros, lc = _kernel_weight(qweight, scales, qzeros, group_size, layout, M, N, K,
                                                 split_k, decode_stream, decode_layout,
                                                 x.dtype == torch.bfloat16)
    x, norm_w = x.contiguous(), norm_w.contiguous()
    if out is None:
        out = torch.empty((M, N), dtype=x.dtype, device=dev)
    else:
        check_out(out, M, N, x)
    ws_bytes = int(lib.awq_w4a16_rmsnorm_gemm_workspace_bytes(M, N, K, int(group_size), int(split_k), lc,
                                                              dtype_code(x.dtype)))
    ws = WORKSPACE.get(dev, ws_bytes)
    rc = lib.awq_w4a16_rmsnorm_gemm(
        _ptr(x), K, _ptr(norm_w), float(eps), _ptr(qweight), _ptr(scales), _ptr(qzeros), _ptr(out),
        int(out.stride(0)), M, N, K, int(group_size), int(split_k), lc, dtype_code(x.dtype),
        dtype_code(norm_w.dtype), dtype_code(scales.dtype), _ptr(ws), ws_bytes, _stream_ptr(dev))
    L.check("awq_w4a16_rmsnorm_gemm", rc)
    return out


# ------------------------------------------------------------------ gated MLP (gate + up)
def gate_up_interleave(gate: torch.Tensor, up: torch.Tensor, half_tile: int) -> torch.Tensor:
    """Two [rows, cols] matrices (2- or 4-byte elements) -> [rows, 2 * ceil(cols / half_tile) *
    half_tile], runs of ``half_tile`` gate elements each followed by the same run of up."""
    lib = L.load()
    _require_device(gate, up)
    if gate.shape != up.shape or gate.dtype != up.dtype or gate.dim() != 2:
        raise ValueError("gate and up must be 2-D tensors of one shape and dtype")
    rows, cols = int(gate.shape[0]), int(gate.shape[1])
    ocols = 2 * (-(-cols // int(half_tile))) * int(half_tile)
    gate, up = gate.contiguous(), up.contiguous()
    out = torch.empty((rows, ocols), dtype=gate.dtype, device=gate.device)
    rc = lib.awq_w4a16_gate_up_interleave(_ptr(gate), _ptr(up), _ptr(out), rows, cols,
                                          int(gate.element_size()), int(half_tile),
                                          _stream_ptr(gate.device))
    L.check("awq_w4a16_gate_up_interleave", rc)
    return out


def _pad_rows(t: torch.Tensor | None, rows: int) -> torch.Tensor | None:
    if t is None or int(t.shape[0]) == rows:
        return t
    pad = torch.zeros((rows - int(t.shape[0]),) + tuple(t.shape[1:]), dtype=t.dtype, device=t.device)
    return torch.cat([t, pad], 0)


def pack_gate_up(gate_qweight, up_qweight, gate_scales, up_scales, gate_qzeros, up_qzeros,
                 group_size: int, layout: str = "ref", kind: str = "autoawq"):
    """The interleaved gate/up matrix of ``gate_up_act``: ``(qweight [K, N/8], scales [K/G, N],
    qzeros [K/G, N/8] or None, derived decode copy or None)``.  ``kind`` "autoawq" or
    "stream" (the decode stream copy) interleave per 64 columns, N = 2 * ceil(I / 64) * 64;
    "narrow" (the narrow decode copy) per 8 columns, N = 2 * ceil(I / 8) * 8.

    ``layout="ref"`` takes the reference's [I, K/8] weights and [I, K/G] scales (I need not be
    a multiple of 8: the missing rows are zero weights with zero scales); "autoawq" takes
    [K, I/8] / [K/G, I]."""
    if layout == "ref":
        i = int(gate_qweight.shape[0])
        i8 = -(-i // 8) * 8
        packed = []
        for qw, sc, qz in ((gate_qweight, gate_scales, gate_qzeros), (up_qweight, up_scales, up_qzeros)):
            packed.append(repack_ref_to_autoawq(_pad_rows(qw.contiguous(), i8), _pad_rows(sc.contiguous(), i8),
                                                _pad_rows(qz.contiguous(), i8) if qz is not None else None,
                                                int(group_size)))
        (gq, gs, gz), (uq, us, uz) = packed
    else:
        gq, gs, gz, uq, us, uz = gate_qweight, gate_scales, gate_qzeros, up_qweight, up_scales, up_qzeros
    wh, sh = (1, 8) if kind == "narrow" else (8, 64)
    qw = gate_up_interleave(gq, uq, wh)
    sc = gate_up_interleave(gs, us, sh)
    qz = gate_up_interleave(gz, uz, wh) if gz is not None else None
    derived = {"stream": pack_decode_stream, "narrow": pack_decode_narrow}.get(kind)
    return qw, sc, qz, (derived(qw) if derived else None)


GATE_UP_CACHE = _DerivedCache("gate_up_pair", pack_gate_up)

GATE_UP_ACTIVATIONS = {"silu": L.MOE_ACT_SILU, "gelu": L.MOE_ACT_GELU_TANH,
                       "gelu_pytorch_tanh": L.MOE_ACT_GELU_TANH}


def gate_up_act(x: torch.Tensor, gate_qweight: torch.Tensor, up_qweight: torch.Tensor,
                gate_scales: torch.Tensor, up_scales: torch.Tensor, group_size: int,
                gate_qzeros: torch.Tensor | None = None, up_qzeros: torch.Tensor | None = None,
                activation: str = "silu", layout: str = "ref", out: torch.Tensor | None = None,
                split_k: int = 0, decode_layout: str | None = None) -> torch.Tensor:
    """``out[M, I] = act(x @ Wg^T) * (x @ Wu^T)`` in one launch of a decode kernel with its
    gated epilogue (M <= 32).  ``activation``: "gelu" / "gelu_pytorch_tanh" select GELU (tanh
    form), anything else SiLU, as the reference decides (awq_fused_gemm.py:3040-3041).  The
    interleaved weight pair is built once and cached.  ``decode_layout``: "narrow", "stream"
    or None (chosen by shape, as for ``gemm``)."""
    lib = L.load()
    if x.dim() != 2:
        raise ValueError("x must be 2-D")
    dev = _require_device(x, gate_qweight, up_qweight, gate_scales, up_scales, gate_qzeros, up_qzeros, out)
    if (gate_qzeros is None) != (up_qzeros is None):
        raise ValueError("gate and up zeros must both be given or both be None")
    M, K = int(x.shape[0]), int(x.shape[1])
    if layout == "ref":
        I, kw = int(gate_qweight.shape[0]), int(gate_qweight.shape[1]) * 8
    else:
        kw, I = int(gate_qweight.shape[0]), int(gate_qweight.shape[1]) * 8
    if kw != K:
        raise ValueError(f"K mismatch: x has {K}, weights have {kw}")
    act = GATE_UP_ACTIVATIONS.get(str(activation).lower(), L.MOE_ACT_SILU)
    if decode_layout not in (None, "narrow", "stream"):
        raise ValueError(f"unknown decode_layout {decode_layout!r}")
    kind = "autoawq"
    if K % 32 == 0 and M <= DECODE_MAX_M:
        n_narrow = 2 * (-(-I // 8)) * 8
        narrow = decode_layout == "narrow" or (decode_layout is None and
                                               _narrow_fits(M, n_narrow, K, int(split_k), x.dtype == torch.bfloat16))
        kind = "narrow" if narrow else "stream"
    qw, sc, qz, st = GATE_UP_CACHE.get(gate_qweight, up_qweight, gate_scales, up_scales, gate_qzeros,
                                       up_qzeros, args=(int(group_size), layout, kind))
    lc = {"narrow": L.LAYOUT_DECODE_NARROW, "stream": L.LAYOUT_DECODE_STREAM}.get(kind, L.LAYOUT_AUTOAWQ)
    if st is not None:
        qw = st
    x = x if x.stride(1) == 1 and x.stride(0) % 8 == 0 else x.contiguous()
    if out is None:
        out = torch.empty((M, I), dtype=x.dtype, device=dev)
    else:
        check_out(out, M, I, x)
    ws_bytes = int(lib.awq_w4a16_gate_up_workspace_bytes(M, I, K, int(group_size), int(split_k), lc))
    ws = WORKSPACE.get(dev, ws_bytes) if ws_bytes else None
    rc = lib.awq_w4a16_gate_up_act(
        _ptr(x), int(x.stride(0)), _ptr(qw), _ptr(sc), _ptr(qz), _ptr(out), int(out.stride(0)), M, I, K,
        int(group_size), int(split_k), lc, act, dtype_code(x.dtype), dtype_code(sc.dtype), _ptr(ws),
        ws_bytes if ws is not None else 0, _stream_ptr(dev))
    L.check("awq_w4a16_gate_up_act", rc)
    return out


# ------------------------------------------------------------------ mixture of experts
MOE_ACTIVATIONS = {"silu": L.MOE_ACT_SILU, "swish": L.MOE_ACT_SILU,
                   "gelu": L.MOE_ACT_GELU_TANH, "gelu_pytorch_tanh": L.MOE_ACT_GELU_TANH}


def moe_route(gating_output: torch.Tensor, topk: int, renormalize: bool = True, *, flow: str = "fp32",
              weights_dtype: torch.dtype | None = None, clamp: bool | None = None):
    """softmax -> top-k -> renormalise on the device: ``(weights, ids int32)``, each ``[T, topk]``;
    equal probabilities select the lower expert id first.

    ``flow="fp32"``: the Gemma4 router (``models/gemma4/moe.py:106-123``): fp32 softmax and
    renormalisation by ``max(sum, 1e-8)`` (``clamp``, default on), weights in ``weights_dtype``
    (default fp32; the router casts them to the hidden dtype).  ``flow="logits"``: ``fused_moe``
    (``fused_moe.py:12-15``): the softmax rounded to the logits dtype, top-k on those values,
    renormalisation in that dtype without a clamp; weights default to the logits dtype."""
    lib = L.load()
    dev = _require_device(gating_output)
    if gating_output.dim() != 2:
        raise ValueError("gating_output must be [T, E]")
    if flow not in ("fp32", "logits"):
        raise ValueError(f"unknown routing flow {flow!r}")
    g = gating_output if gating_output.stride(1) == 1 else gating_output.contiguous()
    T, E = int(g.shape[0]), int(g.shape[1])
    in_dt = flow == "logits"
    if weights_dtype is None:
        weights_dtype = g.dtype if in_dt else torch.float32
    if clamp is None:
        clamp = not in_dt
    flags = (L.ROUTE_RENORMALIZE if renormalize else 0) | (L.ROUTE_SOFTMAX_IN_LOGITS_DTYPE if in_dt else 0)
    flags |= L.ROUTE_CLAMP_SUM if (clamp and renormalize) else 0
    w = torch.empty((T, int(topk)), dtype=weights_dtype, device=dev)
    ids = torch.empty((T, int(topk)), dtype=torch.int32, device=dev)
    rc = lib.awq_w4a16_moe_route_ex(_ptr(g), int(g.stride(0)), dtype_code(g.dtype), T, E, int(topk), flags,
                                    _ptr(w), dtype_code(weights_dtype), _ptr(ids), _stream_ptr(dev))
    L.check("awq_w4a16_moe_route_ex", rc)
    return w, ids


def pack_moe_stream(qweight: torch.Tensor, gate_up: bool) -> torch.Tensor:
    """AutoAWQ expert stack [E, K, N/8] -> the MoE stream layout (int32, flat).  For the
    gate_up stack (N = 2I) each tile pairs gate and up columns."""
    lib = L.load()
    _require_device(qweight)
    if qweight.dtype != torch.int32 or qweight.dim() != 3:
        raise ValueError("expert qweight must be a 3-D int32 tensor [E, K, N/8]")
    e, k, n = int(qweight.shape[0]), int(qweight.shape[1]), int(qweight.shape[2]) * 8
    nbytes = int(lib.awq_w4a16_moe_stream_bytes(e, k, n, 1 if gate_up else 0))
    if nbytes <= 0:
        raise ValueError(f"no MoE stream layout for E={e}, K={k}, N={n}")
    qweight = qweight.contiguous()
    out = torch.empty(nbytes // 4, dtype=torch.int32, device=qweight.device)
    rc = lib.awq_w4a16_moe_pack_stream(_ptr(qweight), _ptr(out), e, k, n, 1 if gate_up else 0,
                                       _stream_ptr(qweight.device))
    L.check("awq_w4a16_moe_pack_stream", rc)
    return out


MOE_STREAM_CACHE = _DerivedCache("moe_stream", pack_moe_stream)


def prepare_moe_stream(qweight: torch.Tensor, gate_up: bool) -> torch.Tensor:
    """Build (and hold on the stack tensor) the MoE stream copy of an AutoAWQ expert stack."""
    return MOE_STREAM_CACHE.get(qweight, args=(bool(gate_up),))


def repack_experts_ref_to_autoawq(qweight: torch.Tensor, scales: torch.Tensor,
                                  qzeros: torch.Tensor | None, group_size: int):
    """Reference expert stacks [E, N, K/8] -> AutoAWQ stacks [E, K, N/8] (lossless)."""
    outs = [repack_ref_to_autoawq(qweight[e], scales[e], qzeros[e] if qzeros is not None else None,
                                  group_size) for e in range(int(qweight.shape[0]))]
    qw = torch.stack([o[0] for o in outs])
    sc = torch.stack([o[1] for o in outs])
    qz = torch.stack([o[2] for o in outs]) if qzeros is not None else None
    return qw, sc, qz


def moe(x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor,
        gate_up_qweight: torch.Tensor, gate_up_scales: torch.Tensor, gate_up_qzeros: torch.Tensor | None,
        down_qweight: torch.Tensor, down_scales: torch.Tensor, down_qzeros: torch.Tensor | None,
        group_size: int, activation: str = "silu", out: torch.Tensor | None = None) -> torch.Tensor:
    """Grouped AWQ MoE on AutoAWQ expert stacks: gate_up [E, H, 2I/8], down [E, I, H/8]
    (scales and zeros in the matching AutoAWQ layouts; zeros None for symmetric z = 8).

    ``out[t] = sum_j w[t, j] * down_e(act(gate_e(x_t)) * up_e(x_t))``, e = ``topk_ids[t, j]``.
    """
    lib = L.load()
    dev = _require_device(x, topk_weights, topk_ids, gate_up_qweight, gate_up_scales, gate_up_qzeros,
                          down_qweight, down_scales, down_qzeros, out)
    if x.dim() != 2:
        raise ValueError("x must be [T, H]")
    if (gate_up_qzeros is None) != (down_qzeros is None):
        raise ValueError("gate_up and down zeros must both be given or both be None")
    try:
        act = MOE_ACTIVATIONS[str(activation).strip().lower()]
    except KeyError:
        raise ValueError(f"unsupported activation {activation!r}") from None
    T, H = int(x.shape[0]), int(x.shape[1])
    E = int(gate_up_qweight.shape[0])
    I = int(gate_up_qweight.shape[2]) * 4
    if int(gate_up_qweight.shape[1]) != H or tuple(down_qweight.shape) != (E, I, H // 8):
        raise ValueError(f"expert stacks do not match H={H}, I={I}, E={E}")
    topk = int(topk_ids.shape[1])
    if tuple(topk_weights.shape) != (T, topk) or tuple(topk_ids.shape) != (T, topk):
        raise ValueError("topk_weights / topk_ids must be [T, top_k]")
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError("topk_ids must be int32 or int64")
    x = x if x.stride(1) == 1 else x.contiguous()
    topk_ids, topk_weights = topk_ids.contiguous(), topk_weights.contiguous()
    gu_sc, dn_sc = gate_up_scales.contiguous(), down_scales.contiguous()
    gu_qz = gate_up_qzeros.contiguous() if gate_up_qzeros is not None else None
    dn_qz = down_qzeros.contiguous() if down_qzeros is not None else None
    gu = prepare_moe_stream(gate_up_qweight, True)
    dn = prepare_moe_stream(down_qweight, False)
    if out is None:
        out = torch.empty((T, H), dtype=x.dtype, device=dev)
    else:
        check_out(out, T, H, x)
    if T == 0:
        return out
    ws_bytes = int(lib.awq_w4a16_moe_workspace_bytes(T, H, I, E, topk))
    ws = WORKSPACE.get(dev, ws_bytes, key="moe")
    rc = lib.awq_w4a16_moe(
        _ptr(x), int(x.stride(0)), _ptr(topk_ids), 64 if topk_ids.dtype == torch.int64 else 32,
        _ptr(topk_weights), dtype_code(topk_weights.dtype), _ptr(gu), _ptr(gu_sc), _ptr(gu_qz), _ptr(dn),
        _ptr(dn_sc), _ptr(dn_qz), _ptr(out), int(out.stride(0)), T, H, I, E, topk, int(group_size), act,
        dtype_code(x.dtype), dtype_code(gu_sc.dtype), _ptr(ws), ws_bytes, _stream_ptr(dev))
    L.check("awq_w4a16_moe", rc)
    return out
