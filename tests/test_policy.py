"""The AWQ execution policy of ``AWQWeight`` / ``PackedInt4Weight`` (CPU only): the reference's
``tests/test_awq_fused_scope_policy.py:27-150`` ported (the process-environment parts become the
tuning snapshot, which is the only place this build reads such knobs), and the first-call decision
of ``matmul`` (``vllm/model_executor/layers/quantization/tensor.py:1008-1122, 1170-1451``) with the
GEMM surfaces replaced by recorders, so no kernel runs.
"""
from __future__ import annotations

from types import SimpleNamespace
from unittest.mock import Mock

import pytest
import torch

from litevllm_amd import tensor as TT


def _dummy_inputs():
    x = torch.zeros((1, 128), dtype=torch.bfloat16)
    qweight = torch.zeros((128, 16), dtype=torch.int32)
    scales = torch.ones((128, 4), dtype=torch.float16)
    return x, qweight, scales


@pytest.fixture(autouse=True)
def _fresh():
    TT.set_awq_tensor_tuning_config({})
    TT.reset_awq_runtime_stats()
    yield
    TT.set_awq_tensor_tuning_config({})
    TT.reset_awq_runtime_stats()


# ---- tests/test_awq_fused_scope_policy.py ----
def test_should_allow_awq_fused_respects_attention_only_scope():
    policy = TT.AWQExecutionPolicy(prefer_fused=True, allow_dense_cache=True, cache_scope="all",
                                   fused_scope="attention_only")
    allow_attn, _ = TT.should_allow_awq_fused("model.layers.0.self_attn.q_proj", policy)
    allow_mlp, reason_mlp = TT.should_allow_awq_fused("model.layers.0.mlp.gate_proj", policy)
    assert allow_attn is True
    assert allow_mlp is False
    assert reason_mlp == "fused_scope_attention_only_non_attn"


def test_should_use_awq_fused_path_short_circuits_on_scope_off():
    x, qweight, scales = _dummy_inputs()
    policy = TT.AWQExecutionPolicy(prefer_fused=True, allow_dense_cache=True, cache_scope="all", fused_scope="off")
    use_fused, reason = TT.should_use_awq_fused_path(x=x, qweight=qweight, scales=scales, qzeros=None, group_size=32,
                                                     prefix="model.layers.0.self_attn.q_proj", policy=policy)
    assert use_fused is False
    assert reason == "fused_scope_off"


def test_awq_decode_gemv_helper_prefers_kernel_policy():
    config = SimpleNamespace(kernel_policy={"awq_decode_gemv": True})
    assert TT.awq_decode_gemv_enabled(config) is True
    assert TT.awq_decode_gemv_enabled(None) is False


def test_resolve_awq_execution_policy_prefers_kernel_policy():
    x, _, _ = _dummy_inputs()
    config = SimpleNamespace(kernel_policy={"awq_fused_scope": "all", "awq_fused_gemm": True,
                                            "awq_cache_scope": "attention_only", "awq_dense_fallback_cache": True})
    policy = TT.resolve_awq_execution_policy("model.layers.0.self_attn.q_proj", x, "gemma4_31b_q4", config=config)
    assert policy.prefer_fused is True
    assert policy.allow_dense_cache is True
    assert policy.cache_scope == "attention_only"
    assert policy.fused_scope == "all"


def test_default_awq_dense_fallback_max_gb(monkeypatch):
    monkeypatch.setattr(torch.cuda, "is_available", Mock(return_value=True))
    for gb, want in ((48, 14.0), (288, 14.0), (32, 8.0), (16, 4.0), (8, 2.0)):
        monkeypatch.setattr(torch.cuda, "get_device_properties",
                            Mock(return_value=SimpleNamespace(total_memory=gb * (1024 ** 3))))
        assert TT._default_awq_dense_fallback_max_gb() == want
    monkeypatch.setattr(torch.cuda, "is_available", Mock(return_value=False))
    assert TT._default_awq_dense_fallback_max_gb() == 4.0


def test_packed_int4_weight_matmul_passes_runtime_kernel_policy(monkeypatch):
    """Gemma4-31B's MLP down projection at decode with ``awq_decode_gemv`` and
    ``gemma4_dense_down_proj``: the fused symmetric GEMM receives the runtime config (and no
    policy dict), and the dense fallback is never reached."""
    qweight = torch.zeros((5376, 2688), dtype=torch.int32)
    scales = torch.ones((5376, 672), dtype=torch.float16)
    weight = TT.PackedInt4Weight(qweight, scales, group_size=32, original_shape=(5376, 21504),
                                 prefix="layers.0.mlp.down_proj", profile_hint="gemma4_31b_q4")
    x = torch.zeros((1, 21504), dtype=torch.bfloat16)
    inf_config = SimpleNamespace(kernel_policy={"awq_decode_gemv": True, "gemma4_dense_down_proj": True})
    expected = torch.full((1, 5376), 0.25, dtype=torch.bfloat16)
    seen = {}

    def _fake_safe(a, qweight, scales, group_size, out=None, bias=None, *, config=None, policy=None, layout="ref"):
        seen["config"] = config
        seen["policy"] = policy
        return expected, True, "ok"

    monkeypatch.setattr(TT._AFG, "packed_int4_symmetric_fused_gemm_safe", _fake_safe)

    def _raise_dense(*args, **kwargs):
        raise AssertionError("dense fallback should be bypassed for runtime policy")

    monkeypatch.setattr(TT.PackedInt4Weight, "_slow_matmul_dequant", _raise_dense)
    y = weight.matmul(x, config=inf_config)
    assert torch.equal(y, expected)
    assert seen["config"] is inf_config
    assert seen["policy"] is None


# ---- the first-call decision of matmul, with recorders in place of the GEMMs ----
class _Rec:
    def __init__(self, monkeypatch, used=True):
        self.fused, self.dense = 0, 0
        rec = self

        def fused(self_, x2, bias, config):
            rec.fused += 1
            return torch.zeros((x2.shape[0], 64), dtype=x2.dtype), used, ("ok" if used else "forced")

        def dense(self_, x, bias):
            rec.dense += 1
            return torch.ones((*x.shape[:-1], 64), dtype=x.dtype)

        monkeypatch.setattr(TT.AWQWeight, "_fused", fused)
        monkeypatch.setattr(TT.AWQWeight, "_slow_matmul_dequant", dense)


def _awq_weight(prefix, hint="", symmetric=False, high_fidelity=False):
    # "meta" tensors carry shapes and dtypes only: the capability check passes (not a CPU
    # input, one device) and no kernel can run on them
    qw = torch.empty((64, 16), dtype=torch.int32, device="meta")
    sc = torch.empty((64, 1), dtype=torch.float16, device="meta")
    qz = torch.empty((64, 1), dtype=torch.int32, device="meta")
    if symmetric:
        return TT.PackedInt4Weight(qw, sc, 128, prefix=prefix, profile_hint=hint, high_fidelity=high_fidelity)
    return TT.AWQWeight(qw, sc, qz, 128, prefix=prefix, profile_hint=hint, high_fidelity=high_fidelity)


def _x():
    return torch.empty((2, 128), dtype=torch.float16, device="meta")


@pytest.mark.parametrize("symmetric", [False, True])
def test_unhinted_mlp_projection_runs_dense_by_default(monkeypatch, symmetric):
    """No profile hint, no ``awq_fused_scope``: attention_only, so an MLP projection takes the
    dense path and an attention projection the fused one (tensor.py:437-443)."""
    rec = _Rec(monkeypatch)
    w = _awq_weight("model.layers.0.mlp.gate_proj", symmetric=symmetric)
    for _ in range(2):
        w.matmul(_x())
    assert (rec.fused, rec.dense) == (0, 2)
    ps = TT.get_awq_runtime_prefix_stats()["model.layers.0.mlp.gate_proj"]
    assert ps["decision_dense"] == 1 and ps["reason:fused_scope_attention_only_non_attn"] == 1
    w = _awq_weight("model.layers.0.self_attn.q_proj", symmetric=symmetric)
    w.matmul(_x())
    assert rec.fused == 1


@pytest.mark.parametrize("symmetric", [False, True])
@pytest.mark.parametrize("hint", ["qwen35_9b_awq", "gemma4_31b_q4"])
def test_profile_hint_widens_the_scope(monkeypatch, symmetric, hint):
    rec = _Rec(monkeypatch)
    w = _awq_weight("model.layers.3.mlp.down_proj", hint=hint, symmetric=symmetric)
    w.matmul(_x())
    w.matmul(_x())
    assert (rec.fused, rec.dense) == (2, 0)
    assert TT.get_awq_runtime_prefix_stats()["model.layers.3.mlp.down_proj"]["decision_fused"] == 1


@pytest.mark.parametrize("symmetric", [False, True])
def test_scope_keys_and_force(monkeypatch, symmetric):
    rec = _Rec(monkeypatch)
    pfx = "model.layers.0.mlp.up_proj"
    _awq_weight(pfx, symmetric=symmetric).matmul(_x(), config={"kernel_policy": {"awq_fused_scope": "all"}})
    assert (rec.fused, rec.dense) == (1, 0)
    _awq_weight(pfx, symmetric=symmetric).matmul(
        _x(), config={"kernel_policy": {"awq_fused_scope": "off", "awq_fused_gemm_force": "1"}})
    assert (rec.fused, rec.dense) == (2, 0)
    att = "model.layers.0.self_attn.o_proj"
    _awq_weight(att, symmetric=symmetric).matmul(_x(), config={"kernel_policy": {"awq_fused_scope": "off"}})
    _awq_weight(att, symmetric=symmetric).matmul(_x(), config={"kernel_policy": {"awq_fused_gemm": "false"}})
    # an unknown scope value reads as "all"
    _awq_weight(pfx, symmetric=symmetric).matmul(_x(), config={"kernel_policy": {"awq_fused_scope": "bogus"}})
    assert (rec.fused, rec.dense) == (3, 2)


@pytest.mark.parametrize("symmetric", [False, True])
def test_high_fidelity_layer_and_prefix_match(monkeypatch, symmetric):
    rec = _Rec(monkeypatch)
    att = "model.layers.0.self_attn.q_proj"
    _awq_weight(att, symmetric=symmetric, high_fidelity=True).matmul(_x())
    assert (rec.fused, rec.dense) == (0, 1)
    TT.set_awq_tensor_tuning_config({"FASTINFERENCE_AWQ_HIGH_FIDELITY_PREFIX_MATCH": "1"})
    _awq_weight(att, symmetric=symmetric).matmul(_x())
    _awq_weight("model.layers.0.attn.qkv", symmetric=symmetric).matmul(_x())   # not in the prefix list
    assert (rec.fused, rec.dense) == (1, 2)
    TT.set_awq_tensor_tuning_config({"FASTINFERENCE_AWQ_HIGH_FIDELITY_ALL": "yes"})
    _awq_weight("model.layers.0.attn.qkv", symmetric=symmetric).matmul(_x())
    assert (rec.fused, rec.dense) == (1, 3)


def test_refused_fused_call_keeps_awq_decision_and_drops_packed(monkeypatch):
    """A refused fused call: ``AWQWeight`` keeps its fused decision and falls back per call
    (tensor.py:1034-1092); ``PackedInt4Weight`` freezes the dense path (tensor.py:1392-1408)."""
    rec = _Rec(monkeypatch, used=False)
    att = "model.layers.0.self_attn.q_proj"
    w = _awq_weight(att)
    w.matmul(_x())
    w.matmul(_x())
    assert (rec.fused, rec.dense) == (2, 2) and w._cached_fused_decision is True
    p = _awq_weight(att, symmetric=True)
    p.matmul(_x())
    p.matmul(_x())
    assert (rec.fused, rec.dense) == (3, 4) and p._cached_fused_decision is False


def test_cache_scope_policy():
    x, _, _ = _dummy_inputs()
    mlp, att = "model.layers.0.mlp.gate_proj", "model.layers.0.self_attn.q_proj"
    cfg = {"kernel_policy": {"awq_cache_scope": "attention_only"}}
    assert TT.resolve_awq_execution_policy(mlp, x, config=cfg).allow_dense_cache is False
    assert TT.resolve_awq_execution_policy(att, x, config=cfg).allow_dense_cache is True
    pol = TT.resolve_awq_execution_policy(att, x, config={"kernel_policy": {"awq_cache_scope": "off"}})
    assert pol.allow_dense_cache is False and pol.cache_scope == "off"
    pol = TT.resolve_awq_execution_policy(att, x, config={"kernel_policy": {"awq_dense_fallback_cache": "0"}})
    assert pol.allow_dense_cache is False
    pol = TT.resolve_awq_execution_policy(mlp, x)
    assert pol.allow_dense_cache and pol.cache_scope == "all" and pol.fused_scope == "attention_only"
    assert TT.should_allow_dense_cache(mlp, TT.AWQExecutionPolicy(True, True, "attention_only", "all")) is False
    assert TT.should_allow_dense_cache(att, TT.AWQExecutionPolicy(True, True, "attention_only", "all")) is True
