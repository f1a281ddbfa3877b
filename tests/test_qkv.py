"""Fused QKV projections (``packed_int4_symmetric_fused_qkv_m1/_m2(_safe)``): q | k | v of
symmetric packed int4 weights in one launch.

CPU tests cover the policy switch and the ``_safe`` reasons in the reference's order.  GPU
tests compare against the exact oracle (float64 sums over the unrounded weights ``(q - 8) * s``,
the decode kernels' formulation) to one ulp of the output dtype at ``max(|y|, 1)``, and check
that the fused result equals the three separate GEMMs bit for bit where the tiles line up.
"""
import numpy as np
import pytest
import torch

from oracle import awq_oracle as O

DEV = torch.device("cuda:0")
ON = {"awq_decode_gemv": True}


def _proj(n, k, seed, sdt=torch.float16, g=32):
    rng = np.random.default_rng(seed)
    qw = torch.from_numpy(O.pack_ref(rng.integers(0, 16, size=(n, k), dtype=np.int64)))
    sc = torch.from_numpy(rng.uniform(0.002, 0.02, size=(n, k // g)).astype(np.float32)).to(sdt)
    return qw, sc


def _w(qw, sc, g=32):
    return O.dequant_ref(qw.numpy(), sc.float().numpy(), None, g, out_dtype="float32", zero_point=False)


def _check(y, ye, dtype):
    y = y.float().cpu().numpy().astype(np.float64)
    a = np.maximum(np.abs(ye), 1.0)
    ulp = 2.0 ** (np.floor(np.log2(a)) - (10 if dtype == torch.float16 else 7))
    assert (np.abs(y - ye) / ulp).max() <= 1.0


def test_decode_gemv_policy_default_off():
    import litevllm_amd as A
    assert not A.awq_decode_gemv_enabled()
    assert A.awq_decode_gemv_enabled(policy=ON)
    assert A.awq_decode_gemv_enabled(config={"kernel_policy": {"awq_decode_gemv": "1"}})


def test_qkv_m1_safe_reasons():
    from litevllm_amd import packed_int4_symmetric_fused_qkv_m1_safe as safe
    (qq, qs), (kq, ks), (vq, vs) = _proj(64, 128, 1), _proj(16, 128, 2), _proj(16, 128, 3)
    x = torch.randn(1, 128, dtype=torch.float16)

    def reason(*a, policy=ON):
        return safe(*a, policy=policy)[2]

    assert reason(x, qq, kq, vq, qs, ks, vs, 32, policy=None) == "decode_gemv_disabled"
    assert reason(torch.randn(2, 128, dtype=torch.float16), qq, kq, vq, qs, ks, vs, 32) == "input_not_m1_2d"
    assert reason(x, qq[0], kq, vq, qs, ks, vs, 32) == "qk_weight_not_2d"
    assert reason(x, qq, kq, vq, qs[0], ks, vs, 32) == "qk_scales_not_2d"
    assert reason(x, qq, kq, vq[0], qs, ks, vs, 32) == "v_bad_shape"
    assert reason(x, qq, kq, vq, qs, ks, vs, 64) == "group_size_not_32"
    assert reason(torch.randn(1, 100, dtype=torch.float16), qq, kq, vq, qs, ks, vs, 32) == "k_not_group_aligned"
    assert reason(torch.randn(1, 96, dtype=torch.float16), qq, kq, vq, qs, ks, vs, 32) == "qk_k_mismatch"
    vq2, vs2 = _proj(16, 96, 4)
    assert reason(x, qq, kq, vq2, qs, ks, vs2, 32) == "v_k_mismatch"
    assert reason(x.float(), qq, kq, vq, qs, ks, vs, 32) == "unsupported_dtype_torch.float32"
    out, used, r = safe(x, qq, kq, vq, qs, ks, vs, 32, policy=ON)  # CPU tensors: kernel path declines
    assert (used, r) == (False, "kernel_exception") and out is x


def test_qkv_m2_safe_reasons():
    from litevllm_amd import packed_int4_symmetric_fused_qkv_m2_safe as safe
    (qq, qs), (kq, ks), (vq, vs) = _proj(64, 128, 1), _proj(16, 128, 2), _proj(16, 128, 3)
    x = torch.randn(2, 128, dtype=torch.float16)

    def reason(*a, policy=ON):
        return safe(*a, policy=policy)[2]

    assert reason(x, qq, kq, vq, qs, ks, vs, 32, policy=None) == "decode_gemv_disabled"
    assert reason(x[:1], qq, kq, vq, qs, ks, vs, 32) == "input_not_m2_2d"
    assert reason(x, qq, kq, vq, qs, ks, vs, 64) == "unsupported_group_layout"
    assert reason(x, qq, kq, vq, qs, ks, None, 32) == "v_bad_shape"
    assert reason(x, qq, kq[0], vq, qs, ks, vs, 32) == "tensor_layout_or_device"
    assert reason(torch.randn(2, 96, dtype=torch.float16), qq, kq, vq, qs, ks, vs, 32) == "qk_k_mismatch"
    vq2, vs2 = _proj(16, 96, 4)
    assert reason(x, qq, kq, vq2, qs, ks, vs2, 32) == "v_k_mismatch"


@pytest.mark.gpu
@pytest.mark.parametrize("qn,kn,vn,k", [(2048, 512, 512, 2048), (100, 20, 20, 256), (4096, 1024, 0, 4096),
                                        (8, 8, 8, 32)])
@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_qkv_matches_oracle(qn, kn, vn, k, M, dt):
    import litevllm_amd as A
    print(f"qkv qn={qn} kn={kn} vn={vn} k={k} M={M} {dt}", flush=True)
    (qq, qs), (kq, ks) = _proj(qn, k, qn, dt), _proj(kn, k, kn + 1, dt)
    vq, vs = _proj(vn, k, vn + 2, dt) if vn else (None, None)
    x = torch.randn(M, k, dtype=dt)
    d = lambda t: t.to(DEV) if t is not None else None
    safe = A.packed_int4_symmetric_fused_qkv_m1_safe if M == 1 else A.packed_int4_symmetric_fused_qkv_m2_safe
    y, used, reason = safe(d(x), d(qq), d(kq), d(vq), d(qs), d(ks), d(vs), 32, policy=ON)
    assert used, reason
    torch.cuda.synchronize()
    ws = [_w(qq, qs), _w(kq, ks)] + ([_w(vq, vs)] if vn else [])
    ye = x.double().numpy() @ np.concatenate(ws, 0).astype(np.float64).T
    assert y.shape == (M, qn + kn + vn)
    _check(y, ye, dt)
