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


def _moe_call(lib, **kw):
    p = _fake(4096)
    return lib.awq_w4a16_moe(
        kw.get("x", p), kw.get("ldx", 64), kw.get("ids", p), kw.get("bits", 32), kw.get("rw", p),
        kw.get("rw_dtype", L.DTYPE_F32), kw.get("gq", p), kw.get("gs", p), kw.get("gz", None), kw.get("dq", p),
        kw.get("ds", p), kw.get("dz", None), kw.get("out", p), kw.get("ldo", 64), kw.get("T", 4),
        kw.get("H", 64), kw.get("I", 32), kw.get("E", 4), kw.get("topk", 2), kw.get("G", 32),
        kw.get("act", L.MOE_ACT_SILU), kw.get("act_dtype", L.DTYPE_F16), L.DTYPE_F16, kw.get("ws", None),
        kw.get("ws_bytes", 0), None)


def test_moe_rejects_bad_args_before_any_launch(lib):
    assert _moe_call(lib, x=None) == L.ERR_NULL
    assert _moe_call(lib, gz=_fake()) == L.ERR_NULL           # zeros for gate_up only
    assert _moe_call(lib, act=5) == L.ERR_UNSUPPORTED
    assert _moe_call(lib, G=256) == L.ERR_UNSUPPORTED
    assert _moe_call(lib, bits=16) == L.ERR_UNSUPPORTED
    assert _moe_call(lib, act_dtype=L.DTYPE_F32) == L.ERR_UNSUPPORTED
    assert _moe_call(lib, I=48) == L.ERR_SHAPE                 # I % G
    assert _moe_call(lib, ldx=32) == L.ERR_STRIDE
    assert _moe_call(lib, T=-1) == L.ERR_SHAPE
    assert _moe_call(lib, T=0) == L.OK                         # nothing to do
    # a real workspace pointer, too small
    assert _moe_call(lib, ws=_fake(256), ws_bytes=256) == L.ERR_WORKSPACE


def test_moe_sizes_are_host_only(lib):
    # config 4: E = 64, H = 2048, I = 1024 -> 16 tiles per expert for both stacks
    assert lib.awq_w4a16_moe_stream_bytes(64, 2048, 2048, 1) == 64 * 16 * (2048 // 32) * 2048
    assert lib.awq_w4a16_moe_stream_bytes(64, 1024, 2048, 0) == 64 * 16 * (1024 // 32) * 2048
    # the stream copy is exactly the size of the packed stack when the tiles are full
    assert lib.awq_w4a16_moe_stream_bytes(64, 2048, 2048, 1) == 64 * 2048 * 2048 // 2
    assert lib.awq_w4a16_moe_stream_bytes(1, 30, 64, 0) == 0   # K % 32
    R, H, I = 512 * 8, 2048, 1024
    ws = lib.awq_w4a16_moe_workspace_bytes(512, H, I, 64, 8)
    assert ws >= R * I * 2 + R * H * 4 + 64 * R * 4
    assert ws < R * I * 2 + R * H * 4 + 64 * R * 4 + 4096


def test_moe_route_rejects_bad_args(lib):
    p = _fake()
    r = lambda **kw: lib.awq_w4a16_moe_route(
        kw.get("lg", p), kw.get("ld", 8), kw.get("dt", L.DTYPE_F16), kw.get("T", 2), kw.get("E", 8),
        kw.get("k", 2), 1, kw.get("w", p), kw.get("ids", p), None)
    assert r(lg=None) == L.ERR_NULL
    assert r(E=300) == L.ERR_SHAPE
    assert r(k=9) == L.ERR_SHAPE
    assert r(ld=4) == L.ERR_STRIDE
    assert r(dt=9) == L.ERR_UNSUPPORTED
    assert r(T=0) == L.OK


def test_decode_layout_choice():
    """The decode layout rule: narrow 16-column tiles only where measured faster."""
    from litevllm_amd import ops
    cus = L.num_cus()
    assert ops._narrow_fits(1, 4096, 4096, 0) and ops._narrow_fits(1, 32 * cus, 14336, 0)
    assert not ops._narrow_fits(1, 32 * cus + 16, 14336, 0)
    # activation rows in the kernel's LDS: four tiles per CU at M <= 2 and K <= 4096, three at
    # K <= 8192 (M <= 4), else two
    assert ops._narrow_fits(1, 64 * cus, 4096, 0) and not ops._narrow_fits(1, 64 * cus + 16, 4096, 0)
    assert ops._narrow_fits(3, 64 * cus, 4096, 0) and not ops._narrow_fits(4, 64 * cus, 4096, 0)
    assert ops._narrow_fits(5, 48 * cus, 4096, 0) and not ops._narrow_fits(5, 48 * cus + 16, 4096, 0)
    assert ops._narrow_fits(6, 32 * cus, 4096, 0) and not ops._narrow_fits(6, 32 * cus + 16, 4096, 0)
    assert ops._narrow_fits(4, 48 * cus, 4096, 0) and not ops._narrow_fits(4, 48 * cus + 16, 4096, 0)
    assert ops._narrow_fits(1, 48 * cus, 8192, 0) and not ops._narrow_fits(1, 48 * cus + 16, 8192, 0)
    assert not ops._narrow_fits(1, 4096, 4096, 2)          # an explicit split asks for the stream kernel
    assert ops._narrow_fits(4, 16 * cus, 4096, 0) and ops._narrow_fits(4, 16 * cus, 14336, 0)
    assert not ops._narrow_fits(4, 16 * cus, 16384, 0) and not ops._narrow_fits(4, 16 * cus + 16, 8192, 0)
    assert ops._narrow_fits(8, 16 * cus, 8192, 0) and not ops._narrow_fits(8, 16 * cus, 12288, 0)
    assert not ops._narrow_fits(16, 16 * cus + 16, 4096, 0) and not ops._narrow_fits(17, 4096, 4096, 0)
    # M = 5 .. 8: two tiles per CU at K <= 4096, one beyond (the M <= 16 rule)
    assert ops._narrow_fits(8, 32 * cus, 4096, 0) and not ops._narrow_fits(8, 32 * cus + 16, 4096, 0)
    assert not ops._narrow_fits(8, 32 * cus, 8192, 0) and ops._narrow_fits(8, 16 * cus, 4096, 0)
    assert not ops._narrow_fits(9, 32 * cus, 4096, 0)
    # bf16 activations: K <= 4096 with one tile per CU up to M = 16, two at M = 1
    assert ops._narrow_fits(1, 32 * cus, 4096, 0, bf16=True) and not ops._narrow_fits(1, 48 * cus, 4096, 0, bf16=True)
    assert not ops._narrow_fits(4, 32 * cus, 4096, 0, bf16=True) and ops._narrow_fits(4, 16 * cus, 4096, 0, bf16=True)
    assert not ops._narrow_fits(1, 16 * cus, 12288, 0, bf16=True) and not ops._narrow_fits(4, 16 * cus, 14336, 0, bf16=True)
    assert ops._narrow_fits(16, 16 * cus, 4096, 0, bf16=True) and not ops._narrow_fits(17, 16 * cus, 4096, 0, bf16=True)


def test_forced_split1_kernel_choice():
    """split_k = 1 keeps auto's kernel wherever auto does not split K (narrow where auto takes
    narrow, the whole-K stream plan where auto's plan has one range), and takes the narrow kernel
    where auto would split: among configs 1 and 2 that is M = 16, N = 6144 and config 2 at
    M = 8 and 32."""
    from litevllm_amd import ops
    if L.num_cus() != 256:
        pytest.skip("planner figures are for a 256-CU part")
    shapes = [(m, 4096, n) for m in (1, 4, 16) for n in (4096, 6144, 24576)] + [(m, 12288, 4096) for m in (1, 8, 32)]
    for M, K, N in shapes:
        auto_narrow = ops._narrow_fits(M, N, K, 0)
        auto_whole_k = auto_narrow or ops._auto_splits(M, N, K) == 1
        forced_narrow = ops._narrow_fits(M, N, K, 1)
        if auto_whole_k:
            assert forced_narrow == auto_narrow, (M, K, N)
        else:
            assert forced_narrow, (M, K, N)
    splitting = [(M, K, N) for M, K, N in shapes if not (ops._narrow_fits(M, N, K, 0) or ops._auto_splits(M, N, K) == 1)]
    assert splitting == [(16, 4096, 6144), (8, 12288, 4096), (32, 12288, 4096)]
    assert ops._auto_splits(1, 24576, 4096) == 1 and ops._auto_splits(16, 6144, 4096) == 4
    assert ops._auto_splits(8, 4096, 12288) == 8


def _rn_gemm(lib, **kw):
    p = _fake(4096)
    return lib.awq_w4a16_rmsnorm_gemm(
        kw.get("x", p), kw.get("ldx", 64), kw.get("nw", p), 1e-6, kw.get("qw", p), kw.get("sc", p), None,
        kw.get("c", p), kw.get("ldc", 64), kw.get("M", 1), kw.get("N", 64), kw.get("K", 64), kw.get("G", 32), 0,
        kw.get("layout", 0), kw.get("act", L.DTYPE_F16), kw.get("ndt", L.DTYPE_F16), L.DTYPE_F16,
        kw.get("ws", p), kw.get("ws_bytes", 0), None)


def test_rmsnorm_rejects_bad_args_before_any_launch(lib):
    p = _fake()
    f = lib.awq_w4a16_rmsnorm
    assert f(p, 64, p, 1e-6, p, 64, 1, 60, L.DTYPE_F16, L.DTYPE_F16, None) == L.ERR_SHAPE  # K % 8
    assert f(p, 64, p, 1e-6, p, 64, -1, 64, L.DTYPE_F16, L.DTYPE_F16, None) == L.ERR_SHAPE
    assert f(p, 64, p, 1e-6, p, 64, 0, 64, L.DTYPE_F16, L.DTYPE_F16, None) == L.OK
    assert f(None, 64, p, 1e-6, p, 64, 1, 64, L.DTYPE_F16, L.DTYPE_F16, None) == L.ERR_NULL
    assert f(p, 64, p, 1e-6, p, 64, 1, 64, L.DTYPE_F32, L.DTYPE_F16, None) == L.ERR_UNSUPPORTED
    assert f(p, 32, p, 1e-6, p, 64, 1, 64, L.DTYPE_F16, L.DTYPE_F16, None) == L.ERR_STRIDE
    assert _rn_gemm(lib, x=None) == L.ERR_NULL
    assert _rn_gemm(lib, ws=None) == L.ERR_WORKSPACE
    assert _rn_gemm(lib, N=60) == L.ERR_SHAPE
    assert _rn_gemm(lib, G=48) == L.ERR_SHAPE
    assert _rn_gemm(lib, layout=9) == L.ERR_UNSUPPORTED
    assert _rn_gemm(lib, ndt=L.DTYPE_F32) == L.ERR_UNSUPPORTED
    assert _rn_gemm(lib, M=0) == L.OK


def test_rmsnorm_gemm_workspace_is_host_only(lib):
    g = lib.awq_w4a16_gemm_workspace_bytes(1, 4096, 12288, 128, 8, 0)
    w16 = lib.awq_w4a16_rmsnorm_gemm_workspace_bytes(1, 4096, 12288, 128, 8, 0, L.DTYPE_F16)
    wbf = lib.awq_w4a16_rmsnorm_gemm_workspace_bytes(1, 4096, 12288, 128, 8, 0, L.DTYPE_BF16)
    assert w16 >= g + 12288 * 2 and wbf >= w16 + 4096 * 2
    # no GEMM workspace (prefill): the counter region is still kept clear
    assert lib.awq_w4a16_gemm_workspace_bytes(256, 4096, 4096, 128, 0, 0) == 0
    assert lib.awq_w4a16_rmsnorm_gemm_workspace_bytes(256, 4096, 4096, 128, 0, 0, L.DTYPE_F16) == 65536 + 256 * 4096 * 2
    # M = 64 runs as two 32-row decode chunks, one after another: one chunk's workspace
    assert lib.awq_w4a16_gemm_workspace_bytes(64, 4096, 4096, 128, 0, 0) == lib.awq_w4a16_gemm_workspace_bytes(32, 4096, 4096, 128, 0, 0)


def test_workspace_grows_geometrically():
    """Split-K / MoE workspaces are kept alive once handed out (graphs captured earlier hold their
    addresses), so they grow in powers of two: requests rising in small steps leave retired
    buffers that add up to less than the live one."""
    import torch
    from litevllm_amd import ops
    ws = ops._Workspace()
    dev = torch.device("cpu")
    for i in range(48):
        n = (16 << 20) + 1 + i * (3 << 20)
        buf = ws.get(dev, n)
        assert buf.numel() >= n and buf.numel() & (buf.numel() - 1) == 0
    live = ws.get(dev, 1).numel()
    assert live == 256 << 20 and len(ws._retired) == 3   # 32, 64 and 128 MiB
    assert sum(int(r.numel()) for r in ws._retired) < live


def test_probe_read_rejects_bad_args_before_any_launch(lib):
    """The read-ceiling probe checks its sizes on the host: nothing is launched for these."""
    p = _fake()
    f = lib.awq_w4a16_probe_read
    assert f(None, 64, 1, 64, 2, p, None) == L.ERR_NULL
    assert f(p, 64, 1, 64, 2, None, None) == L.ERR_NULL
    assert f(p, 0, 1, 64, 2, p, None) == L.ERR_SHAPE
    assert f(p, 72, 1, 64, 2, p, None) == L.ERR_SHAPE      # not a multiple of 16
    assert f(p, 64, 0, 64, 2, p, None) == L.ERR_SHAPE
    assert f(p, 64, 1, 96, 2, p, None) == L.ERR_SHAPE      # threads not a multiple of 64
    assert f(p, 64, 1, 2048, 2, p, None) == L.ERR_SHAPE
    assert f(p, 64, 1, 64, 3, p, None) == L.ERR_UNSUPPORTED
