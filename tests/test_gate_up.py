"""Dense fused gate/up with the activation epilogue: ``act(x @ Wg^T) * (x @ Wu^T)``.

CPU tests cover the oracle, the policy switches, the ``_safe`` reasons in the reference's
order and the caller's structural refusals.  GPU tests run the HIP decode kernel with its
gated epilogue through the C ABI and compare against ``oracle.gate_up_exact`` over the
unrounded weights ``(q - 8) * s`` (float64 sums): every element within one ulp of the output
dtype of the exact value, ulp taken at max(|y|, 1) (fp32 accumulation plus one rounding), and
the reference tests' own
bar (cosine > 0.999, relative MAE < 0.02 against bf16-rounded dense weights,
``tests/test_gemma4_mlp_pair_fusion.py:260-356``).
"""
import types

import numpy as np
import pytest
import torch

from oracle import awq_oracle as O

DEV = torch.device("cuda:0")
ON = {"awq_fused_gate_up": True}


def _pair(n, k, g=32, seed=0, sdt=torch.bfloat16, zero_scale_cols=()):
    """Reference-layout symmetric pair: qweight [n, k/8] int32, scales [n, k/g]."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(2):
        q = rng.integers(0, 16, size=(n, k), dtype=np.int64)
        qw = torch.from_numpy(O.pack_ref(q))
        sc = torch.from_numpy(rng.uniform(0.002, 0.02, size=(n, k // g)).astype(np.float32)).to(sdt)
        for c in zero_scale_cols:
            sc[c] = 0
        out.append((qw, sc))
    return out


def _exact(x, pair, g, activation):
    (qg, sg), (qu, su) = pair
    wg = O.dequant_ref(qg.numpy(), sg.float().numpy(), None, g, out_dtype="float32", zero_point=False)
    wu = O.dequant_ref(qu.numpy(), su.float().numpy(), None, g, out_dtype="float32", zero_point=False)
    return O.gate_up_exact(x.float().cpu().numpy(), wg, wu, activation)


def _ulp(y, dtype):
    # ulp at max(|y|, 1), as the GEMM tests take it: the fp32 sums carry an absolute error of
    # order eps32 * sum|x * w|, which a gate near zero (cancellation) turns into many ulps of a
    # tiny output, in the reference's kernel as in this one
    a = np.maximum(np.abs(y), 1.0)
    e = np.floor(np.log2(a))
    return 2.0 ** (e - (10 if dtype == torch.float16 else 7))


def _check(y, ye, dtype, what):
    y = y.float().cpu().numpy().astype(np.float64)
    err = np.abs(y - ye) / _ulp(ye, dtype)
    assert err.max() <= 1.0, (what, float(err.max()))


# ---------------------------------------------------------------- oracle (CPU)
def test_gate_up_exact_matches_library_routines():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(3, 40, dtype=torch.float64, generator=g)
    wg = torch.randn(24, 40, dtype=torch.float64, generator=g) * 0.2
    wu = torch.randn(24, 40, dtype=torch.float64, generator=g) * 0.2
    F = torch.nn.functional
    want = F.silu(F.linear(x, wg)) * F.linear(x, wu)
    assert np.allclose(O.gate_up_exact(x.numpy(), wg.numpy(), wu.numpy(), "silu"), want.numpy(),
                       rtol=1e-12, atol=1e-14)
    want = F.gelu(F.linear(x, wg), approximate="tanh") * F.linear(x, wu)
    for name in ("gelu", "gelu_pytorch_tanh", "GELU"):
        assert np.allclose(O.gate_up_exact(x.numpy(), wg.numpy(), wu.numpy(), name), want.numpy(),
                           rtol=1e-12, atol=1e-14)
    # the reference maps every other name to SiLU (awq_fused_gemm.py:3040-3041)
    assert np.array_equal(O.gate_up_exact(x.numpy(), wg.numpy(), wu.numpy(), "relu"),
                          O.gate_up_exact(x.numpy(), wg.numpy(), wu.numpy(), "silu"))


def test_gate_up_exact_identity_weights():
    x = np.linspace(-3, 3, 64).reshape(1, 64)
    eye = np.eye(64)
    assert np.allclose(O.gate_up_exact(x, eye, eye, "silu"), x / (1 + np.exp(-x)) * x, rtol=1e-14)
    assert np.allclose(O.gate_up_exact(x, eye, 2 * eye, "silu"), 2 * x * x / (1 + np.exp(-x)), rtol=1e-14)


# ---------------------------------------------------------------- surfaces (CPU)
def test_policy_switches_default_off():
    import litevllm_amd as A
    assert not A.awq_fused_gate_up_enabled()
    assert not A.awq_fused_gate_up_group32_enabled()
    assert A.awq_fused_gate_up_enabled(policy={"awq_fused_gate_up": True})
    assert A.awq_fused_gate_up_enabled(policy={"awq_fused_gate_up": "yes"})
    assert not A.awq_fused_gate_up_enabled(policy={"awq_fused_gate_up": "0"})
    assert A.awq_fused_gate_up_group32_enabled(config={"kernel_policy": {"awq_fused_gate_up_group32": "1"}})
    cfg = types.SimpleNamespace(kernel_policy={"awq_fused_gate_up": "on"})
    assert A.awq_fused_gate_up_enabled(config=cfg)


def test_safe_reasons_in_reference_order():
    from litevllm_amd.awq_fused_gemm import packed_int4_symmetric_fused_gate_up_m1_safe as safe
    (qg, sg), (qu, su) = _pair(64, 128)
    x = torch.randn(1, 128, dtype=torch.bfloat16)

    def reason(*a, policy=ON, **kw):
        return safe(*a, policy=policy, **kw)[2]

    assert reason(x, qg, qu, sg, su, 32, policy=None) == "disabled"
    assert reason(torch.randn(2, 128, dtype=torch.bfloat16), qg, qu, sg, su, 32) == "input_not_m1_2d"
    assert reason(x[0], qg, qu, sg, su, 32) == "input_not_m1_2d"
    assert reason(x, qg[0], qu, sg, su, 32) == "qweight_not_2d"
    assert reason(x, qg, qu, sg[0], su, 32) == "scales_not_2d"
    assert reason(x, qg, qu[:32], sg, su, 32) == "qweight_shape_mismatch"
    assert reason(x, qg, qu, sg, su[:32], 32) == "scale_shape_mismatch"
    assert reason(x.float(), qg, qu, sg, su, 32) == "unsupported_dtype_torch.float32"
    assert reason(x, qg, qu, sg, su, 64) == "group_size_not_32"
    assert reason(torch.randn(1, 96, dtype=torch.bfloat16), qg, qu, sg, su, 32) == "k_mismatch"
    # CPU tensors reach the runner, which needs the GPU library path: reported, not raised
    out, used, r = safe(x, qg, qu, sg, su, 32, policy=ON)
    assert (used, r) == (False, "kernel_exception") and out is x


def test_m1_validation_messages():
    import litevllm_amd as A
    (qg, sg), (qu, su) = _pair(64, 128)
    x = torch.randn(1, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="requires M == 1"):
        A.packed_int4_symmetric_fused_gate_up_m1(torch.randn(2, 128), qg, qu, sg, su, 32)
    with pytest.raises(ValueError, match="requires group_size=32"):
        A.packed_int4_symmetric_fused_gate_up_m1(x, qg, qu, sg, su, 64)
    with pytest.raises(ValueError, match="qweight shape mismatch"):
        A.packed_int4_symmetric_fused_gate_up_m1(x, qg, qu[:8], sg, su, 32)
    with pytest.raises(ValueError, match="scale shape mismatch"):
        A.packed_int4_symmetric_fused_gate_up_m1(x, qg, qu, sg, su[:8], 32)
    with pytest.raises(ValueError, match="K mismatch"):
        A.packed_int4_symmetric_fused_gate_up_m1(torch.randn(1, 96), qg, qu, sg, su, 32)
    with pytest.raises(ValueError, match="group32 fused gate/up requires M=1"):
        A.packed_int4_symmetric_fused_gate_up_group32_m1(torch.randn(2, 128), qg, qu, sg, su, 32)


def _proj(qw, sc, n, k, g=32, **kw):
    d = dict(input_size=k, output_size=n, qweight=qw, scales=sc, qzeros=None, group_size=g, bias=None)
    d.update(kw)
    return types.SimpleNamespace(**d)


def test_caller_refusals():
    from litevllm_amd import try_fused_awq_gate_up_activation as fuse
    (qg, sg), (qu, su) = _pair(64, 128)
    gp, up = _proj(qg, sg, 64, 128), _proj(qu, su, 64, 128)
    x = torch.randn(1, 128, dtype=torch.bfloat16)
    cfg = {"kernel_policy": ON}
    assert fuse(x, gp, up, activation="silu") is None  # policy off by default
    assert fuse(x, gp, up, activation="silu", inf_config=cfg, lora_mapping=[1]) is None
    assert fuse(x, gp, _proj(qu, su, 64, 128, bias=torch.zeros(64)), activation="silu", inf_config=cfg) is None
    assert fuse(x, gp, _proj(qu, su, 64, 128, qzeros=torch.ones(64, 1, dtype=torch.int32)),
                activation="silu", inf_config=cfg) is None
    assert fuse(x, gp, _proj(qu, su, 64, 128, group_size=64), activation="silu", inf_config=cfg) is None
    assert fuse(x, gp, _proj(qu, su, 64, 128, force_high_fidelity_awq=True), activation="silu",
                inf_config=cfg) is None
    assert fuse(torch.randn(2, 128, dtype=torch.bfloat16), gp, up, activation="silu", inf_config=cfg) is None
    # CPU tensors: the kernel path declines, the caller falls back
    assert fuse(x, gp, up, activation="silu", inf_config=cfg) is None


# ---------------------------------------------------------------- GPU parity
REF_CASES = [  # the reference tests' shapes (test_gemma4_mlp_pair_fusion.py:260-356) and more
    (257, 288, "silu", torch.bfloat16),
    (193, 256, "gelu_pytorch_tanh", torch.bfloat16),
    (257, 288, "silu", torch.float16),
    (704, 2816, "silu", torch.bfloat16),       # the reference benchmark's default shape
    (704, 2816, "gelu_pytorch_tanh", torch.float16),
    (14336, 4096, "silu", torch.float16),
    (8, 32, "silu", torch.float16),
    (64, 4096, "gelu", torch.bfloat16),
]


@pytest.mark.gpu
@pytest.mark.parametrize("n,k,act,dt", REF_CASES)
@pytest.mark.parametrize("group32", [False, True])
def test_fused_gate_up_m1_matches_oracle(n, k, act, dt, group32):
    from litevllm_amd.awq_fused_gemm import packed_int4_symmetric_fused_gate_up_m1_safe as safe
    print(f"gate_up n={n} k={k} act={act} dtype={dt} group32={group32}", flush=True)
    pair = _pair(n, k, seed=n + k, sdt=dt)
    (qg, sg), (qu, su) = pair
    x = torch.randn(1, k, dtype=dt)
    pol = dict(ON, awq_fused_gate_up_group32=group32)
    y, used, reason = safe(x.to(DEV), qg.to(DEV), qu.to(DEV), sg.to(DEV), su.to(DEV), 32, activation=act,
                           policy=pol)
    assert used, reason
    torch.cuda.synchronize()
    assert y.shape == (1, n) and y.dtype == dt
    ye = _exact(x, pair, 32, act)
    _check(y, ye, dt, (n, k, act))
    # the reference tests' bar, against bf16-rounded dense weights through torch
    F = torch.nn.functional
    wg = O.dequant_ref(qg.numpy(), sg.float().numpy(), None, 32, out_dtype="float32", zero_point=False)
    wu = O.dequant_ref(qu.numpy(), su.float().numpy(), None, 32, out_dtype="float32", zero_point=False)
    wg, wu = torch.from_numpy(wg).to(dt).float(), torch.from_numpy(wu).to(dt).float()
    a = F.linear(x.float(), wg)
    ref = (F.gelu(a, approximate="tanh") if act.startswith("gelu") else F.silu(a)) * F.linear(x.float(), wu)
    yf = y.float().cpu()
    cos = F.cosine_similarity(yf.reshape(-1), ref.reshape(-1), dim=0).item()
    rel_mae = ((yf - ref).abs().mean() / ref.abs().mean().clamp_min(1e-6)).item()
    assert cos > 0.999 and rel_mae < 0.02, (cos, rel_mae)


@pytest.mark.gpu
@pytest.mark.parametrize("n,k", [(704, 2816), (257, 288), (1000, 1536), (8, 32)])
@pytest.mark.parametrize("M", [1, 4, 17])
@pytest.mark.parametrize("layout", ["narrow", "stream"])
def test_gate_up_act_both_decode_layouts(n, k, M, layout):
    """The gated epilogue of both decode kernels: 16-column narrow tiles (pair interleaved per
    8 columns) and 128-column stream tiles (per 64)."""
    from litevllm_amd import ops
    print(f"gate_up_act layout={layout} n={n} k={k} M={M}", flush=True)
    for dt in (torch.bfloat16, torch.float16):
        pair = _pair(n, k, seed=n + M, sdt=dt)
        (qg, sg), (qu, su) = pair
        x = torch.randn(M, k, dtype=dt)
        y = ops.gate_up_act(x.to(DEV), qg.to(DEV), qu.to(DEV), sg.to(DEV), su.to(DEV), 32,
                            activation="gelu_pytorch_tanh", decode_layout=layout)
        torch.cuda.synchronize()
        _check(y, _exact(x, pair, 32, "gelu_pytorch_tanh"), dt, (layout, n, k, M, dt))


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 3, 16, 17, 32])
@pytest.mark.parametrize("split_k", [0, 1, 3, 7])
def test_gate_up_act_rows_and_splits(M, split_k):
    """More tokens (the decode kernel's one- and two-tile paths) and forced K partitions
    (the split epilogue reduces gate and up partials in split order)."""
    from litevllm_amd import ops
    n, k = 1000, 1536
    print(f"gate_up_act M={M} split_k={split_k}", flush=True)
    for dt in (torch.float16, torch.bfloat16):
        pair = _pair(n, k, seed=M * 10 + split_k, sdt=dt)
        (qg, sg), (qu, su) = pair
        x = torch.randn(M, k, dtype=dt)
        y = ops.gate_up_act(x.to(DEV), qg.to(DEV), qu.to(DEV), sg.to(DEV), su.to(DEV), 32,
                            activation="silu", split_k=split_k)
        torch.cuda.synchronize()
        _check(y, _exact(x, pair, 32, "silu"), dt, (M, split_k, dt))


@pytest.mark.gpu
@pytest.mark.parametrize("G", [64, 128])
def test_gate_up_act_autoawq_with_zeros(G):
    """The C ABI's general form: AutoAWQ [K, I/8] inputs with zero points, larger groups."""
    from litevllm_amd import ops
    from oracle.gen import make_awq_problem
    k, n = 2048, 768
    pg = make_awq_problem(M=2, K=k, N=n, group_size=G, seed=1)
    pu = make_awq_problem(M=2, K=k, N=n, group_size=G, seed=2)
    print(f"gate_up_act autoawq zeros G={G}", flush=True)
    t = lambda a: torch.from_numpy(a).to(DEV)
    y = ops.gate_up_act(t(pg["x"]), t(pg["qweight"]), t(pu["qweight"]), t(pg["scales"]), t(pu["scales"]), G,
                        gate_qzeros=t(pg["qzeros"]), up_qzeros=t(pu["qzeros"]), activation="gelu",
                        layout="autoawq")
    torch.cuda.synchronize()
    wg = O.dequant_awq(pg["qweight"], pg["scales"], pg["qzeros"], G, out_dtype="float32")
    wu = O.dequant_awq(pu["qweight"], pu["scales"], pu["qzeros"], G, out_dtype="float32")
    _check(y, O.gate_up_exact(pg["x"], wg.T, wu.T, "gelu"), torch.float16, G)


@pytest.mark.gpu
def test_gate_up_interleave_layout():
    from litevllm_amd import ops
    g = torch.arange(5 * 20, dtype=torch.int32).reshape(5, 20)
    u = -g - 1
    out = ops.gate_up_interleave(g.to(DEV), u.to(DEV), 8).cpu()
    want = torch.zeros(5, 2 * 3 * 8, dtype=torch.int32)
    for b in range(3):
        for w in range(8):
            c = b * 8 + w
            if c < 20:
                want[:, 16 * b + w] = g[:, c]
                want[:, 16 * b + 8 + w] = u[:, c]
    assert torch.equal(out, want)
    s = torch.randn(3, 100, dtype=torch.float16)
    out = ops.gate_up_interleave(s.to(DEV), (2 * s).to(DEV), 64).cpu()
    assert out.shape == (3, 256)
    assert torch.equal(out[:, :64], s[:, :64]) and torch.equal(out[:, 64:128], 2 * s[:, :64])
    assert torch.equal(out[:, 128:164], s[:, 64:]) and torch.equal(out[:, 192:228], 2 * s[:, 64:])
    assert not out[:, 164:192].any() and not out[:, 228:].any()
