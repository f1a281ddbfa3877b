"""try_fused_awq_pair_matmul: the fusion rules of _fused_awq_pair.py:61-166 (CPU), and the
fused GEMM against the oracle and against the two projections run separately (GPU)."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch
import torch.nn as nn

from litevllm_amd.fused_pair import _lora_is_active, try_fused_awq_pair_matmul
from oracle import awq_oracle as O
from oracle.gen import make_awq_problem
from kernel_paths import decode_serves


def _lin(p, layout="autoawq", dev="cpu", bias=None, zeros=True, **kw):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    K = p["qweight"].shape[0]
    N = p["qweight"].shape[1] * 8
    # a profiled model's MLP pair: the execution policy's fused scope is "all" (tensor.py:437-443)
    return SimpleNamespace(input_size=K, output_size=N, qweight=t(p["qweight"]), scales=t(p["scales"]),
                           qzeros=t(p["qzeros"]) if zeros else None, group_size=p["group_size"],
                           bias=bias, layout=layout, prefix="model.layers.0.mlp.gate_proj",
                           awq_profile_hint="qwen35_9b_awq", **kw)


def test_lora_activity_rules():
    assert not _lora_is_active(None)
    assert not _lora_is_active([None, None])
    assert _lora_is_active([None, 3])
    assert _lora_is_active(SimpleNamespace(adapter_count=1))
    assert not _lora_is_active(SimpleNamespace(adapter_count=0))


def test_unfusable_pairs_return_none():
    pa = make_awq_problem(1, 128, 64, 64, seed=1)
    pb = make_awq_problem(1, 128, 64, 64, seed=2)
    pc = make_awq_problem(1, 128, 128, 64, seed=3)
    x = torch.zeros(1, 128, dtype=torch.float16)
    own = nn.Module()
    a, b = _lin(pa), _lin(pb)
    assert try_fused_awq_pair_matmul(x, a, _lin(pc), own, "k") is None            # output sizes
    assert try_fused_awq_pair_matmul(x, a, b, own, "k", lora_mapping=[1]) is None  # LoRA active
    assert try_fused_awq_pair_matmul(x, a, _lin(pb, bias=torch.zeros(64)), own, "k") is None
    assert try_fused_awq_pair_matmul(x, a, _lin(pb, force_high_fidelity_awq=True), own, "k") is None
    assert try_fused_awq_pair_matmul(x, a, _lin(pb, zeros=False), own, "k") is None  # mixed zeros
    assert try_fused_awq_pair_matmul(x, a, _lin(pb, layout="ref"), own, "k") is None
    assert not hasattr(own, "_fused_awq_pair_k")


@pytest.mark.gpu
@pytest.mark.parametrize("M,zeros", [(1, True), (4, True), (64, True), (16, False)])
def test_fused_pair_matches_oracle_and_separate_calls(M, zeros):
    from litevllm_amd import ops
    K, N, G = 512, 256, 128
    pa = make_awq_problem(M, K, N, G, seed=10 + M)
    pb = make_awq_problem(M, K, N, G, seed=20 + M)
    ba = torch.randn(N, generator=torch.Generator().manual_seed(M)).half()
    bb = torch.randn(N, generator=torch.Generator().manual_seed(M + 1)).half()
    a = _lin(pa, dev="cuda:0", bias=ba.cuda(), zeros=zeros)
    b = _lin(pb, dev="cuda:0", bias=bb.cuda(), zeros=zeros)
    x = torch.from_numpy(pa["x"]).cuda()
    own = nn.Module()
    y = try_fused_awq_pair_matmul(x, a, b, own, "gu")
    assert y is not None and tuple(y.shape) == (M, 2 * N)
    assert hasattr(own, "_fused_awq_pair_gu")
    y2 = try_fused_awq_pair_matmul(x, a, b, own, "gu")   # cached fused weight
    assert torch.equal(y, y2)
    za = pa["qzeros"] if zeros else None
    zb = pb["qzeros"] if zeros else None
    # the skinny kernels (M <= 32, and 32-row chunks of them up to 64) multiply unrounded weights, the prefill one fp16 ones
    wdt = "float32" if decode_serves(M, 2 * N, G) else "float16"
    wa = O.dequant_awq(pa["qweight"], pa["scales"], za, G, out_dtype=wdt, zero_point=zeros)
    wb = O.dequant_awq(pb["qweight"], pb["scales"], zb, G, out_dtype=wdt, zero_point=zeros)
    w = np.concatenate([wa, wb], axis=1).T                       # [2N, K]
    exact = O.linear_exact(pa["x"], w, np.concatenate([ba.numpy(), bb.numpy()]))
    rep = O.error_report(y.cpu().numpy(), exact)
    assert rep["max_ulp"] <= 1.0 and rep["mean_rel"] <= 1e-3, rep
    sep = torch.cat([ops.gemm(x, a.qweight, a.scales, a.qzeros, G, bias=a.bias, layout="autoawq"),
                     ops.gemm(x, b.qweight, b.scales, b.qzeros, G, bias=b.bias, layout="autoawq")], 1)
    rep2 = O.error_report(y.cpu().numpy(), sep.cpu().numpy())
    assert rep2["max_ulp"] <= 1.0, rep2
