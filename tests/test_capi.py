"""CPU-side checks of the C ABI: the built library loads, exports every symbol the header
declares with the expected constants, and rejects bad arguments before touching a GPU."""
import ctypes
import os
import re

import pytest

from litevllm_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "awq_w4a16.h")


def _header():
    with open(HEADER) as f:
        return f.read()


def _declared_functions():
    txt = re.sub(r"/\*.*?\*/", "", _header(), flags=re.S)
    return sorted(set(re.findall(r"\b(awq_w4a16_\w+)\s*\(", txt)))


def _declared_constants():
    return {m.group(1): int(m.group(2)) for m in re.finditer(r"#define\s+(AWQ_\w+)\s+(\d+)", _header())}


@pytest.fixture(scope="module")
def lib():
    if not os.path.isfile(L.LIB_PATH):
        pytest.fail(f"{L.LIB_PATH} missing: run __graft_entry__.build() first")
    return L.load()


def test_every_declared_symbol_is_exported(lib):
    names = _declared_functions()
    assert names, "no declarations parsed"
    for n in names:
        assert hasattr(lib, n), n
        assert n in L.SIGNATURES, f"{n} has no ctypes signature"
    assert set(L.SIGNATURES) == set(names)


def test_python_constants_match_header():
    c = _declared_constants()
    assert c["AWQ_LAYOUT_AUTOAWQ"] == L.LAYOUT_AUTOAWQ
    assert c["AWQ_LAYOUT_KN_SEQ"] == L.LAYOUT_KN_SEQ
    assert c["AWQ_LAYOUT_NK_SEQ"] == L.LAYOUT_NK_SEQ
    for name in ("F16", "BF16", "F32", "NONE"):
        assert c[f"AWQ_DTYPE_{name}"] == getattr(L, f"DTYPE_{name}")
    for name in ("NULL", "SHAPE", "UNSUPPORTED", "WORKSPACE", "LAUNCH", "STRIDE"):
        assert c[f"AWQ_ERR_{name}"] == getattr(L, f"ERR_{name}")


def test_version_and_strerror(lib):
    assert lib.awq_w4a16_version() >= 100
    for code in range(0, 8):
        assert isinstance(lib.awq_w4a16_strerror(code), bytes)
    assert lib.awq_w4a16_strerror(0) == b"ok"


def _fake(n=64):
    # host buffers only stand in for non-NULL pointers; every call below must be
    # rejected by argument validation before any device access
    return ctypes.cast(ctypes.create_string_buffer(n), ctypes.c_void_p).value


def test_gemm_rejects_null_and_bad_shapes(lib):
    p = _fake()
    args = dict(lda=64, M=1, N=64, K=64, G=32)
    g = lambda **kw: lib.awq_w4a16_gemm(
        kw.get("a", p), kw.get("lda", 64), kw.get("qw", p), kw.get("sc", p), None, None,
        kw.get("c", p), kw.get("ldc", 64), kw.get("M", 1), kw.get("N", 64), kw.get("K", 64),
        kw.get("G", 32), 0, kw.get("layout", L.LAYOUT_AUTOAWQ), kw.get("act", L.DTYPE_F16),
        L.DTYPE_F16, L.DTYPE_NONE, None, 0, None)
    assert g(a=None) == L.ERR_NULL
    assert g(c=None) == L.ERR_NULL
    assert g(N=60) == L.ERR_SHAPE                # N % 8
    assert g(G=16) == L.ERR_SHAPE                # group % 32
    assert g(K=96, G=64) == L.ERR_SHAPE          # K % G
    assert g(act=L.DTYPE_F32) == L.ERR_UNSUPPORTED
    assert g(lda=32) == L.ERR_STRIDE
    assert g(layout=7) in (L.ERR_UNSUPPORTED, L.ERR_STRIDE)
    assert g(M=0) == L.OK                        # empty problem: nothing to launch


def test_dequant_rejects_bad_args(lib):
    p = _fake()
    assert lib.awq_w4a16_dequant(None, p, None, p, 8, 8, 8, 0, L.DTYPE_F16, L.DTYPE_F16, None) == L.ERR_NULL
    assert lib.awq_w4a16_dequant(p, p, None, p, 8, 12, 8, 0, L.DTYPE_F16, L.DTYPE_F16, None) == L.ERR_SHAPE
    assert lib.awq_w4a16_dequant(p, p, None, p, 8, 8, 8, 0, L.DTYPE_F32, L.DTYPE_F16, None) == L.ERR_UNSUPPORTED
    assert lib.awq_w4a16_dequant(p, p, None, p, 0, 8, 8, 0, L.DTYPE_F16, L.DTYPE_F16, None) == L.OK


def test_workspace_planning_is_host_only(lib):
    # no split for prefill shapes, fp32 partials + counters for forced decode splits
    assert lib.awq_w4a16_gemm_workspace_bytes(2048, 4096, 4096, 128, 0, 0) == 0
    ws1 = lib.awq_w4a16_gemm_workspace_bytes(1, 4096, 12288, 128, 1, 0)
    ws8 = lib.awq_w4a16_gemm_workspace_bytes(1, 4096, 12288, 128, 8, 0)
    assert ws1 == 0
    assert ws8 >= 8 * 1 * 4096 * 4
