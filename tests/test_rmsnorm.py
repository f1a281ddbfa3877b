"""Fused RMSNorm + int4 GEMM (``rmsnorm_awq_fused_linear``, ``vllm/kernels/triton/
rmsnorm_awq_fused.py:43-189``).

The reference has no tests of its own for this kernel (no caller either).  GPU tests compare
the normalised rows with the pinned oracle (``oracle.awq_oracle.rmsnorm_rows``) bit for bit
(both round an fp64 sum of the exact squares once to fp32), then the product with the exact
oracle on the device's own normalised rows to one ulp of the output at ``max(|y|, 1)`` (the
GEMM kernels' bar), and the whole call with the reference's formulation (oracle rows,
fp16-rounded weights) to one ulp plus a per-output bound of the two known differences: the
decode kernels (M <= 32, and 32-row chunks a little above) multiply by the unrounded weights, as the reference's own M = 1
GEMM does (``awq_fused_gemm.py:1966-1971``), and a normalised element may sit one fp16 ulp
from the oracle's.  bf16 results are the fp16 result converted once, which adds half a bf16
ulp (four fp16 ulps) to each bound.
"""
import numpy as np
import pytest
import torch

from oracle import awq_oracle as O
from kernel_paths import decode_serves

DEV = torch.device("cuda:0")


def _problem(M, N, K, G, seed, dt=torch.float16, ndt=None):
    rng = np.random.default_rng(seed)
    qw = torch.from_numpy(O.pack_ref(rng.integers(0, 16, (N, K))))
    qz = torch.from_numpy(O.pack_ref(rng.integers(0, 16, (N, -(-(K // G) // 8) * 8))))
    sc = torch.from_numpy((np.abs(rng.standard_normal((N, K // G))) * 0.02 + 1e-4).astype(np.float16))
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, K, generator=g) * 2).to(dt)
    nw = (1 + 0.3 * torch.randn(K, generator=g)).to(ndt or dt)
    return x, nw, qw, sc, qz


def _ulps(y, ye, floor=1.0):
    return np.abs(np.asarray(y, np.float64) - ye) / O.fp16_ulp(ye, floor)


def _np(t):
    return t.float().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("M,K", [(1, 8), (1, 4096), (3, 2816), (64, 4096), (5, 12288)])
@pytest.mark.parametrize("dt,ndt", [(torch.float16, torch.float16), (torch.bfloat16, torch.bfloat16),
                                    (torch.float16, torch.bfloat16)])
def test_rmsnorm_rows_vs_oracle(M, K, dt, ndt):
    from litevllm_amd import ops
    print(f"rmsnorm rows M={M} K={K} {dt} {ndt}", flush=True)
    x, nw, *_ = _problem(M, 8, K, 8, M * 7 + K, dt, ndt)
    got = ops.rmsnorm(x.to(DEV), nw.to(DEV), 1e-6).cpu().numpy()
    want = O.rmsnorm_rows(_np(x), _np(nw), 1e-6)
    # the device adds the exact squares in fp64 and rounds once, as the oracle does: bit-exact
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,G", [(1, 6144, 4096, 128), (1, 5632, 2048, 128), (4, 4096, 4096, 128),
                                     (16, 1024, 4096, 64), (32, 512, 12288, 128), (64, 1024, 4096, 128),
                                     (2, 200, 1024, 32)])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_rmsnorm_awq_fused_linear_vs_oracle(M, N, K, G, dt):
    import litevllm_amd as A
    from litevllm_amd import ops
    print(f"rmsnorm gemm M={M} N={N} K={K} G={G} {dt}", flush=True)
    x, nw, qw, sc, qz = _problem(M, N, K, G, 1000 + M + N, dt)
    d = lambda t: t.to(DEV)
    y = A.rmsnorm_awq_fused_linear(d(x), d(qw), d(sc), d(qz), G, d(nw), eps=1e-6)
    torch.cuda.synchronize()
    assert y.dtype == dt and y.shape == (M, N)
    xn = ops.rmsnorm(d(x), d(nw), 1e-6).cpu().numpy()
    w = O.dequant_ref(qw.numpy(), sc.float().numpy(), qz.numpy(), G, out_dtype="float32" if decode_serves(M, N, G) else "float16")
    exact = O.linear_exact(xn, w)
    yv = _np(y.cpu())
    ref = O.rmsnorm_awq_linear(_np(x), _np(nw), 1e-6, qw.numpy(), sc.numpy(), qz.numpy(), G)
    conv = 0.0 if dt == torch.float16 else 4.0  # fp16 -> bf16: half a bf16 ulp = 4 fp16 ulps
    assert _ulps(yv, exact).max() <= 1.0 + conv
    # against the reference's own formulation: within one ulp plus the two documented
    # differences, bounded term by term -- unrounded weights on the decode kernels (each fp16 weight is
    # within 2^-11 of the product, relatively) and a normalised element one fp16 ulp apart
    xo = O.rmsnorm_rows(_np(x), _np(nw), 1e-6).astype(np.float64)
    w16 = np.abs(O.dequant_ref(qw.numpy(), sc.numpy(), qz.numpy(), G).astype(np.float64))
    dev_terms = (np.abs(xo) * 2.0 ** -11 if decode_serves(M, N, G) else 0.0) + O.fp16_ulp(xo, floor=2.0 ** -14)
    bound = dev_terms @ w16.T
    excess = np.abs(yv.astype(np.float64) - ref) - bound
    assert (excess / O.fp16_ulp(ref, 1.0)).max() <= 1.0 + conv


@pytest.mark.gpu
@pytest.mark.parametrize("decode_layout,split_k", [("narrow", 0), ("stream", 0), ("stream", 4), (None, 1)])
def test_rmsnorm_gemm_layouts_agree(decode_layout, split_k):
    """Every decode weight copy and split gives the exact oracle's result to one ulp, and a
    fixed split is bitwise reproducible."""
    from litevllm_amd import ops
    print(f"rmsnorm gemm layout={decode_layout} split={split_k}", flush=True)
    M, N, K, G = 2, 2048, 4096, 128
    x, nw, qw, sc, qz = _problem(M, N, K, G, 77)
    d = lambda t: t.to(DEV)
    y1 = ops.rmsnorm_gemm(d(x), d(nw), 1e-6, d(qw), d(sc), d(qz), G, split_k=split_k, decode_layout=decode_layout)
    y2 = ops.rmsnorm_gemm(d(x), d(nw), 1e-6, d(qw), d(sc), d(qz), G, split_k=split_k, decode_layout=decode_layout)
    assert torch.equal(y1, y2)
    xn = ops.rmsnorm(d(x), d(nw), 1e-6).cpu().numpy()
    exact = O.linear_exact(xn, O.dequant_ref(qw.numpy(), sc.float().numpy(), qz.numpy(), G, out_dtype="float32"))
    assert _ulps(_np(y1.cpu()), exact).max() <= 1.0


def test_rmsnorm_awq_fused_linear_rejects_bad_inputs():
    import litevllm_amd as A
    x, nw, qw, sc, qz = _problem(1, 16, 64, 32, 1)
    with pytest.raises(ValueError):
        A.rmsnorm_awq_fused_linear(x[0], qw, sc, qz, 32, nw)
    with pytest.raises(ValueError):
        A.rmsnorm_awq_fused_linear(x.float(), qw, sc, qz, 32, nw)
    with pytest.raises(ValueError):
        A.rmsnorm_awq_fused_linear(x[:, :32], qw, sc, qz, 32, nw)


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,G,ndt", [(1, 6144, 4096, 128, torch.float16), (3, 4096, 2816, 64, torch.bfloat16),
                                         (4, 1000, 1024, 32, torch.float16), (1, 8, 256, 128, torch.bfloat16)])
@pytest.mark.parametrize("zp", [True, False])
def test_rmsnorm_prologue_in_narrow_kernel_matches_two_launches(M, N, K, G, ndt, zp):
    """The narrow kernel's own prologue (one fp16 row: one launch) gives the same bits as the
    separate row-norm launch followed by the narrow GEMM; several rows take the two launches,
    and both are held to the exact oracle."""
    from litevllm_amd import ops
    print(f"rmsnorm narrow prologue M={M} N={N} K={K} G={G} {ndt} zp={zp}", flush=True)
    x, nw, qw, sc, qz = _problem(M, N, K, G, 500 + M + K, torch.float16, ndt)
    d = lambda t: t.to(DEV) if t is not None else None
    qz = qz if zp else None
    fused = ops.rmsnorm_gemm(d(x), d(nw), 1e-6, d(qw), d(sc), d(qz), G, decode_layout="narrow")
    xn = ops.rmsnorm(d(x), d(nw), 1e-6)
    two = ops.gemm(xn, d(qw), d(sc), d(qz), G, decode_layout="narrow")
    assert torch.equal(fused, two)
    w = O.dequant_ref(qw.numpy(), sc.float().numpy(), qz.numpy() if zp else None, G, out_dtype="float32",
                      zero_point=zp)
    exact = O.linear_exact(O.rmsnorm_rows(_np(x), _np(nw), 1e-6), w)
    assert _ulps(_np(fused.cpu()), exact).max() <= 1.0
    assert _ulps(_np(two.cpu()), exact).max() <= 1.0
