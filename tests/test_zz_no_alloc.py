"""The allocation-free GEMM entry point (``awq_w4a16_gemm_noalloc``) through the C ABI, against
``awq_w4a16_gemm`` with a caller workspace: the same plan and kernels, so outputs are bitwise
equal (and within 1 fp16 ulp of the exact oracle).  Two calls in a row, the second smaller, both
on split-K plans (the scratch carries counters and partials); a request beyond the fixed scratch
is refused before any launch."""
import numpy as np
import pytest
import torch

from litevllm_amd import _lib as L
from litevllm_amd import ops
from oracle import awq_oracle as O
from oracle.gen import make_awq_problem

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _p(t):
    return None if t is None else int(t.data_ptr())


def _noalloc(lib, x, qw, sc, qz, out, M, N, K, G, split_k, layout):
    return lib.awq_w4a16_gemm_noalloc(_p(x), int(x.stride(0)), _p(qw), _p(sc), _p(qz), None, _p(out),
                                      int(out.stride(0)), M, N, K, G, split_k, layout, L.DTYPE_F16, L.DTYPE_F16,
                                      L.DTYPE_NONE, int(torch.cuda.current_stream().cuda_stream))


@pytest.mark.parametrize("layout", [L.LAYOUT_DECODE_STREAM, L.LAYOUT_AUTOAWQ])
def test_noalloc_matches_gemm_two_calls(layout):
    lib = L.load()
    assert lib.awq_w4a16_gemm_noalloc_max_workspace() == 65536 + (8 << 20)
    # second call smaller than the first; both plans split K (the scratch is used)
    for M, K, N, G in ((16, 4096, 4096, 128), (1, 2048, 1024, 64)):
        print(f"noalloc layout={layout} M={M} K={K} N={N} G={G}", flush=True)
        ws = int(lib.awq_w4a16_gemm_workspace_bytes(M, N, K, G, 0, layout))
        assert ws > 65536, "the plan must split K for this test to exercise the scratch"
        p = make_awq_problem(M=M, K=K, N=N, group_size=G, seed=M + K + N)
        x = torch.from_numpy(p["x"]).to(DEV)
        qw = torch.from_numpy(p["qweight"]).to(DEV)
        sc = torch.from_numpy(p["scales"]).to(DEV)
        qz = torch.from_numpy(p["qzeros"]).to(DEV)
        qk = ops.pack_decode_stream(qw) if layout == L.LAYOUT_DECODE_STREAM else qw
        ref = torch.empty((M, N), dtype=torch.float16, device=DEV)
        wsb = torch.zeros(ws, dtype=torch.uint8, device=DEV)
        rc = lib.awq_w4a16_gemm(_p(x), K, _p(qk), _p(sc), _p(qz), None, _p(ref), N, M, N, K, G, 0, layout,
                                L.DTYPE_F16, L.DTYPE_F16, L.DTYPE_NONE, _p(wsb), ws,
                                int(torch.cuda.current_stream().cuda_stream))
        assert rc == 0
        for _ in range(2):  # and again: the counters are left zero by the previous call
            out = torch.full((M, N), 7.0, dtype=torch.float16, device=DEV)
            assert _noalloc(lib, x, qk, sc, qz, out, M, N, K, G, 0, layout) == 0
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        w = O.dequant_awq(p["qweight"], p["scales"], p["qzeros"], G, out_dtype="float32")
        rep = O.error_report(out.cpu().numpy(), O.linear_exact(p["x"], w.T))
        assert rep["max_ulp"] <= 1.0, rep


def test_noalloc_refuses_beyond_scratch_and_serves_unsplit_calls():
    lib = L.load()
    M, K, N, G = 32, 12288, 24576, 128
    need = int(lib.awq_w4a16_gemm_workspace_bytes(M, N, K, G, 8, L.LAYOUT_DECODE_STREAM))
    assert need > lib.awq_w4a16_gemm_noalloc_max_workspace()
    dummy = torch.zeros(16, dtype=torch.float16, device=DEV)
    rc = lib.awq_w4a16_gemm_noalloc(_p(dummy), K, _p(dummy), _p(dummy), None, None, _p(dummy), N, M, N, K, G, 8,
                                    L.LAYOUT_DECODE_STREAM, L.DTYPE_F16, L.DTYPE_F16, L.DTYPE_NONE,
                                    int(torch.cuda.current_stream().cuda_stream))
    assert rc == L.ERR_WORKSPACE
    # a prefill-shaped call needs no scratch at all
    M, K, N, G = 64, 512, 256, 128
    p = make_awq_problem(M=M, K=K, N=N, group_size=G, seed=9)
    t = {k: torch.from_numpy(v).to(DEV) for k, v in p.items() if isinstance(v, np.ndarray)}
    out = torch.empty((M, N), dtype=torch.float16, device=DEV)
    assert _noalloc(lib, t["x"], t["qweight"], t["scales"], t["qzeros"], out, M, N, K, G, 0, L.LAYOUT_AUTOAWQ) == 0
    ref = ops.gemm(t["x"], t["qweight"], t["scales"], t["qzeros"], G, layout="autoawq")
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
