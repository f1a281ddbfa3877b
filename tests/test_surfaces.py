"""The drop-in Python surfaces the reference's callers bind (survey rows a1, a3, a9, the row-exact
mode and the ``out=`` contract).

CPU part: every ``_safe`` / capability-check reason string in the reference's order
(``vllm/kernels/triton/awq_fused_gemm.py:3713-3831, 2925-2998``,
``vllm/model_executor/layers/quantization/awq_triton.py:7-61``), the geometry inference of
``awq_dequantize_triton`` (``awq_triton.py:150-194``), the ``split_k_iters`` mapping of
``awq_gemm_triton`` (``awq_triton.py:197-209``), the workspace's regrowth rule and the signed
zero-point convention of the loader.  Reasons that need two devices use ``meta`` tensors, which
carry shapes and dtypes but no data, so no kernel can run on them.

GPU part (``-m gpu``): ``AWQConfig.apply`` on reference-layout ``[N, K/8]`` tensors, the dense
fallback after a refused fused call, ``awq_gemm_triton`` with ``split_k_iters`` 1 and 4,
``awq_dequantize_triton`` in both geometries, the row-exact M = 2 / 4 mode (each row bit-equal to
its own M = 1 call, the reference's ``tests/test_awq_fused_gemm_numerics.py:128-161``), and
``out=`` validation before any launch.  Bars as in ``tests/test_gpu_gemm.py``: dequantized
weights bit-exact; GEMM outputs within 1 fp16 ulp (at max(|y|, 1)) of the exact oracle with the
weights the serving kernel multiplies.
"""
import importlib

import numpy as np
import pytest
import torch

from litevllm_amd import ops
from oracle import awq_oracle as O
from oracle.gen import make_awq_problem
from kernel_paths import decode_serves

# the modules themselves (the package re-exports functions of the same names)
AFG = importlib.import_module("litevllm_amd.awq_fused_gemm")
AT = importlib.import_module("litevllm_amd.awq_triton")

DEV = torch.device("cuda:0")


# ------------------------------------------------------------------ CPU: reason strings
def _meta(*shape, dtype=torch.float16):
    return torch.empty(shape, dtype=dtype, device="meta")


def _args(M=2, K=256, N=64, G=128, dev="cpu"):
    a = torch.zeros((M, K), dtype=torch.float16, device=dev)
    qw = torch.zeros((N, K // 8), dtype=torch.int32, device=dev)
    sc = torch.ones((N, K // G), dtype=torch.float16, device=dev)
    qz = torch.zeros((N, max(1, K // G // 8)), dtype=torch.int32, device=dev)
    return a, qw, sc, qz


def test_awq_fused_gemm_safe_reasons_in_reference_order():
    """One failing check at a time, in the reference's order; each call returns (a, False,
    reason) and never raises.  CPU tensors that pass every check reach the launch, which
    refuses them: "kernel_exception"."""
    a, qw, sc, qz = _args()
    f = AFG.awq_fused_gemm_safe
    cases = [
        (dict(a=a[0]), "input_not_2d"),
        (dict(qweight=qw[0]), "qweight_not_2d"),
        (dict(scales=sc[0]), "scales_not_2d"),
        (dict(qzeros=None), "qzeros_bad"),
        (dict(qzeros=qz[0]), "qzeros_bad"),
        (dict(a=torch.zeros((2, 128), dtype=torch.float16)), "k_mismatch"),
        (dict(group_size=0), "group_mismatch"),
        (dict(group_size=96), "group_mismatch"),
        (dict(scales=_meta(64, 2)), "device_mismatch"),
        (dict(qzeros=_meta(64, 1, dtype=torch.int32)), "device_mismatch"),
        (dict(a=a.float()), "unsupported_dtype_torch.float32"),
        (dict(bias=torch.zeros(63)), "bias_bad_shape"),
        (dict(bias=torch.zeros((64, 1))), "bias_bad_shape"),
        (dict(bias=_meta(64)), "bias_device_mismatch"),
        (dict(bias=torch.zeros(64, dtype=torch.int32)), "unsupported_bias_dtype_torch.int32"),
        (dict(out=torch.empty((2, 63), dtype=torch.float16)), "bad_output_shape"),
        (dict(out=torch.empty((2, 64), dtype=torch.float32)), "bad_output"),
        (dict(out=torch.empty((64, 2), dtype=torch.float16).t()), "bad_output"),
        (dict(), "kernel_exception"),
    ]
    for over, want in cases:
        kw = dict(a=a, qweight=qw, scales=sc, qzeros=qz, group_size=128)
        kw.update(over)
        c, used, reason = f(kw.pop("a"), kw.pop("qweight"), kw.pop("scales"), kw.pop("qzeros"), **kw)
        assert (used, reason) == (False, want), (over.keys(), reason)
    # first failing check wins: not 2-D input beats a K mismatch and a bad bias
    _, _, r = f(a[0], qw[:, :3], sc, qz, 128, bias=torch.zeros(3))
    assert r == "input_not_2d"
    _, _, r = f(torch.zeros((2, 128), dtype=torch.float16), qw, sc, qz, 0)
    assert r == "k_mismatch"


def test_symmetric_safe_reasons_in_reference_order():
    a, qw, sc, _ = _args()
    f = AFG.packed_int4_symmetric_fused_gemm_safe
    cases = [
        (dict(a=a[0]), "input_not_2d"),
        (dict(qweight=qw[0]), "qweight_not_2d"),
        (dict(scales=sc[0]), "scales_not_2d"),
        (dict(a=torch.zeros((2, 64), dtype=torch.float16)), "k_mismatch"),
        (dict(group_size=-1), "group_mismatch"),
        (dict(qweight=_meta(64, 32, dtype=torch.int32)), "device_mismatch"),
        (dict(a=a.to(torch.int16)), "unsupported_dtype_torch.int16"),
        (dict(bias=torch.zeros(65)), "bias_bad_shape"),
        (dict(bias=_meta(64)), "bias_device_mismatch"),
        (dict(bias=torch.zeros(64, dtype=torch.float64)), "unsupported_bias_dtype_torch.float64"),
        (dict(), "kernel_exception"),
    ]
    for over, want in cases:
        kw = dict(a=a, qweight=qw, scales=sc, group_size=128)
        kw.update(over)
        _, used, reason = f(kw.pop("a"), kw.pop("qweight"), kw.pop("scales"), **kw)
        assert (used, reason) == (False, want), (over.keys(), reason)


def test_rows_exact_safe_reasons_in_reference_order():
    """``packed_int4_symmetric_group32_rows_exact_msmall_safe`` (awq_fused_gemm.py:2925-2998)."""
    a, qw, sc, _ = _args(M=2, K=256, N=64, G=32)
    f = AFG.packed_int4_symmetric_group32_rows_exact_msmall_safe
    cases = [
        (dict(a=a[0]), "input_not_m2_or_m4_2d"),
        (dict(a=torch.zeros((3, 256), dtype=torch.float16)), "input_not_m2_or_m4_2d"),
        (dict(scales=sc[0]), "weight_or_scales_not_2d"),
        (dict(group_size=128), "unsupported_group_layout"),
        (dict(a=torch.zeros((2, 240), dtype=torch.float16)), "unsupported_group_layout"),
        (dict(a=torch.zeros((4, 128), dtype=torch.float16)), "k_mismatch"),
        (dict(scales=torch.ones((64, 4), dtype=torch.float16)), "scales_shape_mismatch"),
        (dict(scales=_meta(64, 8)), "tensor_device_or_dtype"),
        (dict(a=a.float()), "tensor_device_or_dtype"),
        (dict(bias=torch.zeros(64, dtype=torch.int8)), "bias_layout_or_dtype"),
        (dict(a=torch.zeros((256, 2), dtype=torch.float16).t()), "noncontiguous_input"),
        (dict(out=torch.empty((2, 65), dtype=torch.float16)), "bad_output"),
        (dict(), "kernel_exception"),
    ]
    for over, want in cases:
        kw = dict(a=a, qweight=qw, scales=sc, group_size=32)
        kw.update(over)
        _, used, reason = f(kw.pop("a"), kw.pop("qweight"), kw.pop("scales"), **kw)
        assert (used, reason) == (False, want), (over.keys(), reason)


def test_capability_checks_in_reference_order():
    """``awq_fused_capability_check`` / ``packed_int4_fused_capability_check``
    (awq_triton.py:7-61): the first failing check's reason; "ok" for a valid non-CPU call."""
    ac, qwc, scc, _ = _args()
    a, qw, sc, qz = (t.to("meta") for t in _args())
    f = AT.awq_fused_capability_check
    assert f(a, qw, sc, qz, 128) == (True, "ok")
    assert f(ac, qw, sc, qz, 128) == (False, "cpu_input")
    assert f(a, qwc, sc, qz, 128) == (False, "device_mismatch")
    assert f(a.float(), qw, sc, qz, 128) == (False, "unsupported_input_dtype_torch.float32")
    assert f(a, qw[0], sc, qz, 128) == (False, "qweight_not_2d")
    assert f(a, qw, sc[0], qz, 128) == (False, "scales_not_2d")
    assert f(a, qw, sc, None, 128) == (False, "qzeros_missing")
    assert f(a, qw, sc, qz[0], 128) == (False, "qzeros_not_2d")
    assert f(_meta(2, 128), qw, sc, qz, 128) == (False, "k_dim_mismatch")
    assert f(a, qw, sc, qz, 0) == (False, "bad_group_size")
    assert f(a, qw, sc, qz, 96) == (False, "k_not_divisible_by_group")
    g = AT.packed_int4_fused_capability_check
    assert g(a, qw, sc, 128) == (True, "ok")
    assert g(ac, qw, sc, 128) == (False, "cpu_input")
    assert g(a, qw, scc, 128) == (False, "device_mismatch")
    assert g(a.to(torch.int8), qw, sc, 128) == (False, "unsupported_input_dtype_torch.int8")
    assert g(a, qw, sc, -32) == (False, "bad_group_size")
    assert g(a, qw, sc, 512) == (False, "k_not_divisible_by_group")


def test_dequantize_triton_geometry_inference(monkeypatch):
    """``scales.shape[0] != qweight.shape[0]`` means groups run along the rows (kn_seq), else
    the reference layout (awq_triton.py:161); a failing launch is wrapped as
    RuntimeError("[AWQ_FALLBACK_DEQUANT] ...") (awq_triton.py:190-193)."""
    seen = []
    monkeypatch.setattr(ops, "dequant", lambda *a, layout=None, **k: seen.append(layout) or "sentinel")
    qw = torch.zeros((256, 8), dtype=torch.int32)
    assert AT.awq_dequantize_triton(qw, torch.ones((2, 64)), torch.zeros((2, 8), dtype=torch.int32), 128) == "sentinel"
    assert AT.awq_dequantize_triton(qw, torch.ones((256, 1)), torch.zeros((256, 1), dtype=torch.int32), 64) == "sentinel"
    AT.awq_dequantize_triton(qw, torch.ones((2, 64)), None, 128, layout="autoawq")
    assert seen == ["kn_seq", "ref", "autoawq"]
    monkeypatch.undo()
    with pytest.raises(RuntimeError, match=r"^\[AWQ_FALLBACK_DEQUANT\]"):
        AT.awq_dequantize_triton(qw, torch.ones((2, 64)), torch.zeros((2, 8), dtype=torch.int32), 128)


def test_gemm_triton_split_k_mapping(monkeypatch):
    """``split_k_iters`` 1 leaves the partition to the library (0), > 1 fixes it; leading
    dimensions are flattened and restored; a weight dtype unlike the input's raises, as
    ``matmul`` of mismatched dtypes does in the reference."""
    seen = []

    def fake_gemm(a2, qw, sc, qz, g, split_k=0, layout="ref"):
        seen.append((tuple(a2.shape), split_k, layout))
        return torch.zeros((a2.shape[0], 16))
    monkeypatch.setattr(ops, "gemm", fake_gemm)
    x = torch.zeros((3, 5, 64), dtype=torch.float16)
    y = AT.awq_gemm_triton(x, None, None, None, 32, split_k_iters=1)
    assert y.shape == (3, 5, 16)
    AT.awq_gemm_triton(x, None, None, None, 32, split_k_iters=4)
    AT.awq_gemm_triton(x[0], None, None, None, 32, split_k_iters=0, layout="autoawq")
    assert seen == [((15, 64), 0, "ref"), ((15, 64), 4, "ref"), ((5, 64), 0, "autoawq")]
    with pytest.raises(RuntimeError):
        AT.awq_gemm_triton(x, None, None, None, 32, out_dtype=torch.bfloat16)


def test_out_problem_rules():
    a = torch.zeros((3, 8), dtype=torch.float16)
    assert ops.out_problem(torch.empty((3, 16), dtype=torch.float16), 3, 16, a) is None
    assert ops.out_problem(torch.empty((3, 15), dtype=torch.float16), 3, 16, a) == "bad_output_shape"
    assert ops.out_problem(torch.empty((3, 16), dtype=torch.bfloat16), 3, 16, a) == "bad_output"
    assert ops.out_problem(torch.empty((16, 3), dtype=torch.float16).t(), 3, 16, a) == "bad_output"
    assert ops.out_problem(torch.empty((3, 32), dtype=torch.float16)[:, :16], 3, 16, a) is None
    with pytest.raises(ValueError, match="bad_output_shape"):
        ops.check_out(torch.empty((4, 16), dtype=torch.float16), 3, 16, a)


def test_workspace_regrowth_keeps_old_buffers():
    """A grown workspace never frees the buffer it replaces (graphs captured earlier hold its
    address); a request that fits returns the current buffer."""
    ws = ops._Workspace()
    cpu = torch.device("cpu")
    b1 = ws.get(cpu, 1 << 10)
    assert ws.get(cpu, 2 << 10) is b1          # fits the 16 MiB minimum
    b2 = ws.get(cpu, (16 << 20) + 1)
    assert b2 is not b1 and b2.numel() >= (16 << 20) + 1
    assert any(r is b1 for r in ws._retired)
    assert ws.get(cpu, 10, key="moe") is not b2  # keys are independent buffers
    assert int(b2.sum()) == 0                  # zero-initialised


def test_loader_signed_zero_points():
    """int8 zero points are the signed int4 convention (compressed-tensors: [-8, 7], weights
    offset by +8), mapped to unsigned nibbles by +8; other integer dtypes are unsigned [0, 15];
    out-of-range values raise."""
    from litevllm_amd import loader
    z8 = torch.tensor([[-8, -1, 0, 3, 7]], dtype=torch.int8)
    assert loader.unsigned_zero_points(z8).tolist() == [[0, 7, 8, 11, 15]]
    packed = loader._pack_groups(z8)
    assert O.unpack_ref(packed.numpy())[0, :5].tolist() == [0, 7, 8, 11, 15]
    zu = torch.tensor([[0, 15, 3]], dtype=torch.uint8)
    assert loader.unsigned_zero_points(zu).tolist() == [[0, 15, 3]]
    assert loader.unsigned_zero_points(zu.to(torch.int32)).tolist() == [[0, 15, 3]]
    for bad in (torch.tensor([[8]], dtype=torch.int8), torch.tensor([[-1]], dtype=torch.int32),
                torch.tensor([[16]], dtype=torch.int64)):
        with pytest.raises(ValueError):
            loader.unsigned_zero_points(bad)
    with pytest.raises(ValueError):
        loader.unsigned_zero_points(torch.zeros((1, 2)))
    # q - z is preserved: a signed weight q_s with zero z_s dequantizes like q_s + 8 with z_s + 8
    zs = torch.tensor([[-3, 5]], dtype=torch.int8)
    assert ((torch.tensor([[2, -4]]) + 8) - loader.unsigned_zero_points(zs)).tolist() == [[5, -9]]


# ------------------------------------------------------------------ GPU surfaces
def _ref_layout(p):
    return O.repack_awq_to_ref(p["qweight"], p["qzeros"], p["scales"])


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N,G", [(1, 1024, 512, 128), (3, 2048, 1024, 128), (48, 1024, 768, 64)])
@pytest.mark.parametrize("zp", [True, False])
def test_awqconfig_apply_reference_layout(M, K, N, G, zp):
    """``AWQConfig.apply`` (awq.py:40-104) on a layer holding reference-layout tensors
    (``qweight [N, K/8]``, ``scales [N, K/G]``, ``qzeros [N, K/G/8]``): builds and caches the
    weight object on the first call (AWQWeight with zeros, PackedInt4Weight without), forwards
    ``matmul`` with the layer's bias, and matches the exact oracle."""
    from litevllm_amd.awq import AWQConfig
    from litevllm_amd.tensor import AWQWeight, PackedInt4Weight, reset_awq_runtime_stats, get_awq_runtime_stats
    print(f"AWQConfig.apply M={M} K={K} N={N} G={G} zp={zp}", flush=True)
    p = make_awq_problem(M=M, K=K, N=N, group_size=G, seed=M + K + N)
    qr, zr, sr = _ref_layout(p)
    cfg = AWQConfig.from_config({"quant_method": "awq", "bits": 4, "group_size": G})
    assert cfg.group_size == G and cfg.get_name() == "awq"
    layer = torch.nn.Module()
    cfg.init_layer(layer)
    layer.prefix = "model.layers.0.mlp.down_proj"
    layer.awq_profile_hint = "qwen35_9b_awq"  # a profiled model: fused scope "all" (tensor.py:437-443)
    items = [("model.layers.0.mlp.down_proj.qweight", torch.from_numpy(qr).to(DEV)),
             ("model.layers.0.mlp.down_proj.scales", torch.from_numpy(sr).to(DEV))]
    if zp:
        items.append(("model.layers.0.mlp.down_proj.qzeros", torch.from_numpy(zr).to(DEV)))
    bias = torch.from_numpy(np.random.default_rng(M).standard_normal(N).astype(np.float16))
    items.append(("model.layers.0.mlp.down_proj.bias", bias.to(DEV)))
    cfg.load_weights(layer, iter(items))
    x = torch.from_numpy(p["x"]).to(DEV).view(1, M, K)  # leading dims are kept
    reset_awq_runtime_stats()
    y = cfg.apply(layer, x, inf_config={"kernel_policy": {}})
    assert isinstance(layer._quant_weight, AWQWeight if zp else PackedInt4Weight)
    first = layer._quant_weight
    y2 = cfg.apply(layer, x)
    assert layer._quant_weight is first and torch.equal(y, y2)
    assert y.shape == (1, M, N)
    st = get_awq_runtime_stats()
    # the first call resolves the policy and re-enters, as the reference's does (tensor.py:1121-1122,
    # 1443-1447): three counted entries for two calls
    assert st["awq_fused_success"] == 2 and st["awq_matmul_calls"] == 3
    w = O.dequant_awq(p["qweight"], p["scales"], p["qzeros"] if zp else None, G,
                      out_dtype="float32" if decode_serves(M, N, G) else "float16", zero_point=zp)
    ye = O.linear_exact(p["x"], w.T, bias.double().numpy())
    rep = O.error_report(y.view(M, N).cpu().numpy(), ye)
    assert rep["max_ulp"] <= 1.0, rep


@pytest.mark.gpu
def test_awqconfig_apply_rejects_bad_group_and_unready_layer():
    from litevllm_amd.awq import AWQConfig
    cfg = AWQConfig(group_size=96)
    layer = torch.nn.Module()
    cfg.init_layer(layer)
    x = torch.zeros((1, 256), dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError, match="not ready"):
        cfg.apply(layer, x)
    layer.qweight = torch.nn.Parameter(torch.zeros((64, 32), dtype=torch.int32, device=DEV), requires_grad=False)
    with pytest.raises(RuntimeError, match="group_size=96"):
        cfg.apply(layer, x)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["forced_refusal", "policy_off", "high_fidelity"])
def test_dense_fallback(mode, monkeypatch):
    """The dense path (tensor.py:1053-1092, 1124-1147): HIP dequant (bit-exact) once into the
    LRU, then F.linear; taken after a refused fused call (forced used=False), with the fused
    policy off, or for a high-fidelity layer.  Its output is within the reference-path bar of the
    exact product of the fp16-rounded weights."""
    from litevllm_amd import tensor as TT
    print(f"dense fallback {mode}", flush=True)
    M, K, N, G = 5, 1024, 512, 128
    p = make_awq_problem(M=M, K=K, N=N, group_size=G, seed=77)
    qr, zr, sr = _ref_layout(p)
    w = TT.AWQWeight(torch.from_numpy(qr).to(DEV), torch.from_numpy(sr).to(DEV), torch.from_numpy(zr).to(DEV), G,
                     prefix="fb.self_attn.q_proj", high_fidelity=(mode == "high_fidelity"))
    cfg = None
    if mode == "forced_refusal":
        monkeypatch.setattr(w, "_fused", lambda x2, bias, config: (x2, False, "forced"))
    elif mode == "policy_off":
        cfg = {"kernel_policy": {"awq_fused_gemm": "0"}}
    TT.reset_awq_runtime_stats()
    TT.clear_global_weight_cache()
    x = torch.from_numpy(p["x"]).to(DEV)
    y = w.matmul(x, config=cfg)
    y2 = w.matmul(x, config=cfg)
    assert torch.equal(y, y2)
    ps = TT.get_awq_runtime_prefix_stats()["fb.self_attn.q_proj"]
    # the first call re-enters once its decision is made (not for a high-fidelity layer)
    assert ps["dense_build"] == 1 and ps["cache_hit"] == 1
    assert ps["matmul_calls"] == (2 if mode == "high_fidelity" else 3)
    if mode == "forced_refusal":
        # the decision stays fused (tensor.py:1034-1086): each call tries and falls back
        assert ps["decision_fused"] == 1 and ps["reason:forced"] == 2 and ps["fused_runtime_fallback"] == 2
    elif mode == "policy_off":
        assert ps["decision_dense"] == 1 and ps["reason:fused_disabled"] == 1 and "fused_attempt" not in ps
    else:
        assert ps["high_fidelity_forced"] == 1 and "fused_attempt" not in ps
    wd = w.dense_weight()
    w16 = O.dequant_ref(qr, sr, zr, G)                              # [N, K] fp16, the oracle's dequant
    assert np.array_equal(wd.cpu().numpy().view(np.uint16), w16.view(np.uint16))
    ye = O.linear_exact(p["x"], w16)
    d = np.abs(y.cpu().numpy().astype(np.float64) - ye)
    assert (d <= np.maximum(2e-2, O.fp16_ulp(ye, floor=2.0 ** -14))).all()
    assert d.sum() / np.abs(ye).sum() <= 1e-3
    TT.clear_global_weight_cache()


@pytest.mark.gpu
@pytest.mark.parametrize("split", [1, 4])
@pytest.mark.parametrize("M", [1, 8, 64])
def test_awq_gemm_triton_split_k_iters(M, split):
    """``awq_gemm_triton(input, qweight, scales, zeros, group_size, split_k_iters)`` on
    reference-layout tensors: split 1 and 4 each within 1 ulp of the exact oracle, split 4
    bitwise reproducible (M = 64 runs as two 32-row chunks of the decode kernels)."""
    print(f"awq_gemm_triton M={M} split={split}", flush=True)
    K, N, G = 4096, 1024, 128
    p = make_awq_problem(M=M, K=K, N=N, group_size=G, seed=5 * M + split)
    qr, zr, sr = _ref_layout(p)
    args = (torch.from_numpy(qr).to(DEV), torch.from_numpy(sr).to(DEV), torch.from_numpy(zr).to(DEV))
    x = torch.from_numpy(p["x"]).to(DEV)
    y = AT.awq_gemm_triton(x, *args, group_size=G, split_k_iters=split)
    y2 = AT.awq_gemm_triton(x, *args, group_size=G, split_k_iters=split)
    assert torch.equal(y, y2)
    w = O.dequant_awq(p["qweight"], p["scales"], p["qzeros"], G, out_dtype="float32" if decode_serves(M, N, G) else "float16")
    rep = O.error_report(y.cpu().numpy(), O.linear_exact(p["x"], w.T))
    assert rep["max_ulp"] <= 1.0, rep


@pytest.mark.gpu
@pytest.mark.parametrize("geometry", ["ref", "kn_seq"])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
def test_awq_dequantize_triton_geometries(geometry, out_dtype):
    """Both geometries the reference infers from the scales' rows (awq_triton.py:150-194),
    sequential nibbles in both: bit-exact against one rounding of the exact product."""
    rng = np.random.default_rng(3)
    R, C, G = 256, 512, 64   # unpacked [R, C]; groups run along C (ref) or along R (kn_seq)
    W = rng.integers(0, 16, size=(R, C), dtype=np.int32)
    if geometry == "ref":
        Z = rng.integers(0, 16, size=(R, C // G), dtype=np.int32)
        S = (np.abs(rng.standard_normal((R, C // G))) * 0.02 + 1e-4).astype(np.float16)
        exact = (W.reshape(R, C // G, G) - Z[:, :, None]) * S.astype(np.float64)[:, :, None]
        qz = O.pack_ref(Z) if (C // G) % 8 == 0 else None
    else:
        Z = rng.integers(0, 16, size=(R // G, C), dtype=np.int32)
        S = (np.abs(rng.standard_normal((R // G, C))) * 0.02 + 1e-4).astype(np.float16)
        exact = (W.reshape(R // G, G, C) - Z[:, None, :]) * S.astype(np.float64)[:, None, :]
        qz = O.pack_ref(Z)
    exact = exact.reshape(R, C)
    out = AT.awq_dequantize_triton(torch.from_numpy(O.pack_ref(W)).to(DEV), torch.from_numpy(S).to(DEV),
                                   torch.from_numpy(qz).to(DEV), G, out_dtype=out_dtype).cpu()
    assert out.shape == (R, C)
    want = torch.from_numpy(np.ascontiguousarray(exact)).to(out_dtype)
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("n,k", [(128, 128), (4096, 4096), (24576, 4096), (4096, 14336)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rows_exact_msmall_matches_independent_m1_bitwise(n, k, dtype):
    """The reference's check (tests/test_awq_fused_gemm_numerics.py:128-161): M = 2 and 4
    through ``packed_int4_symmetric_group32_rows_exact_msmall_safe`` equal, bit for bit, the rows
    computed one by one with ``packed_int4_symmetric_fused_gemm`` at M = 1.  Shapes cover the
    narrow copy (N = 4096) and the 128-column stream copy with split-K (N = 24576, K = 14336)."""
    print(f"rows_exact n={n} k={k} {dtype}", flush=True)
    g = torch.Generator().manual_seed(7)
    qweight = torch.randint(-(2**31), 2**31 - 1, (n, k // 8), dtype=torch.int32, generator=g).to(DEV)
    scales = (torch.rand((n, k // 32), generator=g) * 0.02 + 1e-4).to(dtype).to(DEV)
    w = O.dequant_ref(qweight.cpu().numpy(), scales.float().cpu().numpy(), None, 32, out_dtype="float32",
                      zero_point=False).T.astype(np.float64)   # [K, N], unrounded (q - 8) * s
    for m in (2, 4):
        x = torch.randn((m, k), generator=g).to(dtype).to(DEV)
        batched, used, reason = AFG.packed_int4_symmetric_group32_rows_exact_msmall_safe(x, qweight, scales,
                                                                                          group_size=32)
        assert used, reason
        rows = torch.cat([AFG.packed_int4_symmetric_fused_gemm(x[r:r + 1], qweight, scales, group_size=32)
                          for r in range(m)], dim=0)
        assert torch.equal(batched.view(torch.int16), rows.view(torch.int16))
        # and the numbers themselves: within one ulp of the exact sum over unrounded weights
        ye = x.double().cpu().numpy() @ w
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ye), 1.0))) - (10 if dtype == torch.float16 else 7))
        assert (np.abs(batched.float().cpu().numpy() - ye) <= ulp).all()


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N,G,split_k", [(3, 4096, 4096, 128, 0), (7, 4096, 24576, 128, 0), (4, 12288, 4096, 128, 4),
                                             (32, 2048, 1536, 64, 0), (5, 1024, 520, 32, 3), (2, 4096, 24576, 128, 2)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rows_exact_single_launch_zero_point(M, K, N, G, split_k, dtype):
    """``ops.gemm_rows_exact`` (one launch, grid rows = M) on AutoAWQ tensors with zero points and
    a bias: row m equals ``ops.gemm`` of row m alone, bit for bit -- on the narrow copy (N = 4096,
    1536, 520), the stream copy without split (N = 24576) and with forced splits (each grid row
    has counters and partials of its own), for fp16 and bf16, into a row-strided output."""
    print(f"rows_exact single launch M={M} K={K} N={N} G={G} split={split_k} {dtype}", flush=True)
    p = make_awq_problem(M=M, K=K, N=N, group_size=G, seed=M + K + N)
    t = {k: torch.from_numpy(v).to(DEV) for k, v in p.items() if isinstance(v, np.ndarray)}
    x = t["x"].to(dtype)
    sc = t["scales"].to(dtype)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(M)).to(dtype).to(DEV)
    big = torch.zeros((M, N + 64), dtype=dtype, device=DEV)
    out = big[:, :N]
    y = ops.gemm_rows_exact(x, t["qweight"], sc, t["qzeros"], G, bias=bias, split_k=split_k, layout="autoawq", out=out)
    assert y.data_ptr() == out.data_ptr()
    rows = torch.cat([ops.gemm(x[m:m + 1], t["qweight"], sc, t["qzeros"], G, bias=bias, split_k=split_k,
                               layout="autoawq") for m in range(M)])
    assert torch.equal(out.view(torch.int16), rows.view(torch.int16))
    assert bool((big[:, N:] == 0).all())
    # a second call reuses the workspace whose counters the first left at zero
    y2 = ops.gemm_rows_exact(x, t["qweight"], sc, t["qzeros"], G, bias=bias, split_k=split_k, layout="autoawq")
    assert torch.equal(y2.view(torch.int16), rows.view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("N,copies", [(24576, {"ref_scales_zeros", "ref_decode_stream"}),
                                      (4096, {"ref_scales_zeros", "ref_decode_narrow", "ref_decode_stream"})])
def test_weight_holds_its_derived_copies(N, copies):
    """A reference-layout ``AWQWeight`` after decode (M = 1) and prefill (M = 64) calls: its
    qweight parameter holds its derived packs itself -- AutoAWQ scales and zeros, and one kernel
    copy of the int4 weights per kernel family used (the stream copy serves decode and prefill
    at N = 24576; at N = 4096 decode reads the narrow copy) -- and never the repacked AutoAWQ
    qweight.  No module-level table holds any of them; they go with the weight.  Outputs stay
    within 1 ulp of the exact oracle and equal the raw-tensor surface's."""
    import gc
    import weakref
    from litevllm_amd import tensor as TT
    print(f"derived copies N={N}", flush=True)
    K, G = 4096, 128
    p = make_awq_problem(M=64, K=K, N=N, group_size=G, seed=N)
    qr, zr, sr = _ref_layout(p)
    w = TT.AWQWeight(torch.from_numpy(qr).to(DEV), torch.from_numpy(sr).to(DEV), torch.from_numpy(zr).to(DEV), G,
                     prefix="model.layers.0.self_attn.qkv_proj")
    x = torch.from_numpy(p["x"]).to(DEV)
    for m in (1, 64):
        y = w.matmul(x[:m]).cpu().numpy()
        wd = O.dequant_awq(p["qweight"], p["scales"], p["qzeros"], G,
                           out_dtype="float32" if decode_serves(m, N, G) else "float16")
        rep = O.error_report(y, O.linear_exact(p["x"][:m], wd.T))
        assert rep["max_ulp"] <= 1.0, (m, rep)
        y2 = AFG.awq_fused_gemm(x[:m], w.qweight, w.scales, w.qzeros, G)
        assert torch.equal(torch.from_numpy(y), y2.cpu())
    held = ops.derived_copies(w.qweight)
    assert set(held) == copies, sorted(held)
    int4_bytes = K * N // 2
    kernel_copies = [v for k, v in held.items() if k.startswith("ref_decode")]
    assert all(v.numel() * v.element_size() <= int4_bytes * 1.01 for v in kernel_copies)
    assert not any(isinstance(v, dict) and v for c in (ops.STREAM_CACHE, ops.REF_STREAM_CACHE) for v in vars(c).values())
    ref = weakref.ref(held["ref_decode_stream"])
    del held, kernel_copies, w
    gc.collect()
    assert ref() is None  # the copy went with the weight


@pytest.mark.gpu
def test_rows_exact_policy_in_packed_int4_weight():
    """``awq_rows_exact_msmall`` on: PackedInt4Weight.matmul at M = 2 / 4 takes the row-exact
    path (tensor.py:1200-1234) and equals per-row M = 1 calls; off: the generic path."""
    from litevllm_amd import tensor as TT
    n, k = 1024, 2048
    g = torch.Generator().manual_seed(3)
    qweight = torch.randint(-(2**31), 2**31 - 1, (n, k // 8), dtype=torch.int32, generator=g).to(DEV)
    scales = (torch.rand((n, k // 32), generator=g) * 0.02 + 1e-4).half().to(DEV)
    w = TT.PackedInt4Weight(qweight, scales, 32, prefix="rx")
    cfg = {"kernel_policy": {"awq_rows_exact_msmall": True, "awq_fused_scope": "all"}}
    TT.reset_awq_runtime_stats()
    x = torch.randn((4, k), generator=g).half().to(DEV)
    y = w.matmul(x, config=cfg)
    rows = torch.cat([w.matmul(x[r:r + 1], config=cfg) for r in range(4)])
    assert torch.equal(y.view(torch.int16), rows.view(torch.int16))
    assert TT.get_awq_runtime_prefix_stats()["rx"]["rows_exact_msmall_success"] == 1
    # M = 3 is outside the mode: the generic path
    y3 = w.matmul(x[:3], config=cfg)
    assert y3.shape == (3, n) and TT.get_awq_runtime_prefix_stats()["rx"]["rows_exact_msmall_success"] == 1


@pytest.mark.gpu
def test_out_argument_checked_before_launch():
    """A caller-supplied ``out`` of the wrong shape, dtype or stride is refused before any kernel
    writes into it: ``ops.gemm`` raises ValueError and leaves it untouched; the ``_safe`` surface
    returns the reason; a correct ``out`` (also a row-strided view) receives the result."""
    M, K, N, G = 3, 1024, 256, 128
    p = make_awq_problem(M=M, K=K, N=N, group_size=G, seed=4)
    qr, zr, sr = _ref_layout(p)
    t = [torch.from_numpy(v).to(DEV) for v in (qr, sr, zr)]
    x = torch.from_numpy(p["x"]).to(DEV)
    small = torch.full((M, N - 8), 7.0, dtype=torch.float16, device=DEV)
    with pytest.raises(ValueError, match="bad_output_shape"):
        ops.gemm(x, *t, G, out=small)
    assert bool((small == 7.0).all())
    with pytest.raises(ValueError, match="bad_output"):
        ops.gemm(x, *t, G, out=torch.empty((M, N), dtype=torch.float32, device=DEV))
    c, used, reason = AFG.awq_fused_gemm_safe(x, *t, G, out=small)
    assert (used, reason) == (False, "bad_output_shape") and c is x
    big = torch.zeros((M, 2 * N), dtype=torch.float16, device=DEV)
    view = big[:, :N]
    c, used, reason = AFG.awq_fused_gemm_safe(x, *t, G, out=view)
    assert used and reason == "ok"
    ref = ops.gemm(x, *t, G)
    assert torch.equal(big[:, :N], ref) and bool((big[:, N:] == 0).all())
