"""Drop-in for the AWQ weight objects of
``vllm/model_executor/layers/quantization/tensor.py``: ``QuantizedLinearWeight``,
``AWQWeight`` and ``PackedInt4Weight`` keep the ``matmul(x, bias=None, *, config=None)``
protocol (``tensor.py:946-959``), the execution policy (``tensor.py:338-450, 544-673``: fused
scope, cache scope, the force and dense-fallback-cache switches, the profile hint), the frozen
first-call fused/dense decision (``tensor.py:1094-1122``, ``1415-1451``), the dense-weight LRU
fallback (``tensor.py:1085-1092, 1124-1147``) and the runtime counters (``tensor.py:226-243``).

Both paths run on the GPU: the fused path calls the HIP GEMM; the dense fallback
dequantizes with the HIP dequant kernel and multiplies with ``F.linear`` -- exactly the
reference's fallback structure.  Neither has a CPU branch.
"""
from __future__ import annotations

import importlib
from abc import ABC, abstractmethod
from collections import OrderedDict, defaultdict
from dataclasses import dataclass
from typing import Any

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops

# the module, not its functions: a caller (or a test) that replaces a surface of it is seen here
_AFG = importlib.import_module(".awq_fused_gemm", __package__)
_AT = importlib.import_module(".awq_triton", __package__)

_STATS: dict[str, int] = defaultdict(int)
_PREFIX_STATS: dict[str, dict[str, int]] = defaultdict(lambda: defaultdict(int))


def _stat(key: str, delta: int = 1) -> None:
    _STATS[key] += delta


def _prefix_stat(prefix: str, key: str, delta: int = 1) -> None:
    _PREFIX_STATS[prefix or "<unknown>"][key] += delta


def get_awq_runtime_stats() -> dict[str, int]:
    out = dict(_STATS)
    out.update(_GLOBAL_WEIGHT_CACHE.get_memory_stats())
    return out


def get_awq_runtime_prefix_stats() -> dict[str, dict[str, int]]:
    return {k: dict(v) for k, v in _PREFIX_STATS.items()}


def reset_awq_runtime_stats() -> None:
    _STATS.clear()
    _PREFIX_STATS.clear()


class LRUWeightCache:
    """Dense-fallback weight cache bounded by item count and bytes (``tensor.py:60-115``)."""

    def __init__(self, max_size: int = 256, max_bytes: int = 0):
        self.max_size = max_size
        self.max_bytes = max(0, int(max_bytes))
        self.current_bytes = 0
        self._d: OrderedDict[int, torch.Tensor] = OrderedDict()

    def get(self, key: int):
        v = self._d.get(key)
        if v is not None:
            self._d.move_to_end(key)
        return v

    def put(self, key: int, value: torch.Tensor) -> None:
        if key in self._d:
            return
        nb = int(value.numel() * value.element_size())
        if self.max_bytes and nb > self.max_bytes:
            return
        while self._d and ((self.max_size and len(self._d) >= self.max_size)
                           or (self.max_bytes and self.current_bytes + nb > self.max_bytes)):
            _, old = self._d.popitem(last=False)
            self.current_bytes -= int(old.numel() * old.element_size())
        self._d[key] = value
        self.current_bytes += nb

    def get_memory_stats(self) -> dict[str, int]:
        return {"cache_items": len(self._d), "cache_bytes": int(self.current_bytes),
                "cache_max_bytes": int(self.max_bytes), "cache_max_items": int(self.max_size)}

    def clear(self) -> None:
        self._d.clear()
        self.current_bytes = 0


def _default_awq_dense_fallback_max_gb() -> float:
    """Dense-fallback cache budget by device memory (``tensor.py:168-183``): 14 GB from 48 GB
    up, 8 from 32, 4 from 16 (and without a GPU), else 2."""
    if not torch.cuda.is_available():
        return 4.0
    try:
        total_gb = float(torch.cuda.get_device_properties(0).total_memory) / (1024 ** 3)
    except Exception:
        return 4.0
    if total_gb >= 48.0:
        return 14.0
    if total_gb >= 32.0:
        return 8.0
    if total_gb >= 16.0:
        return 4.0
    return 2.0


_GLOBAL_WEIGHT_CACHE = LRUWeightCache(max_size=512, max_bytes=0)


def clear_global_weight_cache() -> None:
    _GLOBAL_WEIGHT_CACHE.clear()


# ---- tuning snapshot (tensor.py:10-31, 120-183): the engine installs it before model load; no
# process environment is read on the hot path ----
_AWQ_TENSOR_TUNING: dict[str, str] = {}
_AWQ_TENSOR_TUNING_LOCKED = False
# the projections the reference keeps on the dense path when prefix matching is switched on
# (tensor.py:200-216)
_DEFAULT_HIGH_FIDELITY_PREFIXES = (
    ".linear_attn.in_proj_qkv", ".linear_attn.in_proj_z", ".linear_attn.in_proj_a", ".linear_attn.in_proj_b",
    ".linear_attn.out_proj", ".self_attn.q_proj", ".self_attn.k_proj", ".self_attn.v_proj", ".self_attn.o_proj",
    ".shared_expert.gate_proj", ".shared_expert.up_proj", ".shared_expert.down_proj", ".mlp.gate_proj",
    ".mlp.up_proj", ".mlp.down_proj",
)
_HIGH_FIDELITY_ALL = False
_HIGH_FIDELITY_PREFIX_MATCH = False
_HIGH_FIDELITY_PREFIXES = _DEFAULT_HIGH_FIDELITY_PREFIXES


def _tuning(name: str, default: str = "") -> str:
    return _AWQ_TENSOR_TUNING.get(name, default)


def _tuning_truthy(name: str, default: str = "0") -> bool:
    return _tuning(name, default).strip().lower() in ("1", "true", "yes", "on")


def _refresh_awq_tuning_derived() -> None:
    """The knobs derived from the snapshot (``tensor.py:120-154``); also empties the dense cache."""
    global _HIGH_FIDELITY_ALL, _HIGH_FIDELITY_PREFIX_MATCH, _HIGH_FIDELITY_PREFIXES
    _HIGH_FIDELITY_ALL = _tuning_truthy("FASTINFERENCE_AWQ_HIGH_FIDELITY_ALL", "0")
    _HIGH_FIDELITY_PREFIX_MATCH = _tuning_truthy("FASTINFERENCE_AWQ_HIGH_FIDELITY_PREFIX_MATCH", "0")
    global _DENSE_BUDGET_SET
    _DENSE_BUDGET_SET = False  # sized at the next dense build (the default asks the device)
    _GLOBAL_WEIGHT_CACHE.clear()
    _HIGH_FIDELITY_PREFIXES = tuple(
        part.strip() for part in _tuning("FASTINFERENCE_AWQ_HIGH_FIDELITY_PREFIXES",
                                         ",".join(_DEFAULT_HIGH_FIDELITY_PREFIXES)).split(",") if part.strip())


_DENSE_BUDGET_SET = False


def _ensure_dense_budget() -> None:
    """The dense cache's byte budget: ``FASTINFERENCE_AWQ_DENSE_FALLBACK_MAX_GB`` of the snapshot,
    else by device memory; none with the legacy cache (``tensor.py:133-145``).  Taken at the first
    dense build rather than at import, so importing the package touches no device."""
    global _DENSE_BUDGET_SET
    if _DENSE_BUDGET_SET:
        return
    raw = _tuning("FASTINFERENCE_AWQ_DENSE_FALLBACK_MAX_GB", "")
    max_gb = float(raw) if raw.strip() else _default_awq_dense_fallback_max_gb()
    legacy = _tuning_truthy("FASTINFERENCE_AWQ_LEGACY_CACHE", "0")
    _GLOBAL_WEIGHT_CACHE.max_bytes = 0 if legacy else int(max_gb * (1024 ** 3))
    _DENSE_BUDGET_SET = True


def set_awq_tensor_tuning_config(values: dict[str, object] | None, *, locked: bool = False) -> None:
    """Install the AWQ execution/cache policy snapshot (``tensor.py:20-31``)."""
    global _AWQ_TENSOR_TUNING, _AWQ_TENSOR_TUNING_LOCKED
    _AWQ_TENSOR_TUNING = {str(k): str(v) for k, v in (values or {}).items() if v is not None}
    _AWQ_TENSOR_TUNING_LOCKED = bool(locked)
    _refresh_awq_tuning_derived()


_refresh_awq_tuning_derived()


# ---- execution policy (tensor.py:53-57, 338-450, 544-673) ----
@dataclass(frozen=True)
class AWQExecutionPolicy:
    prefer_fused: bool
    allow_dense_cache: bool
    cache_scope: str
    fused_scope: str


def _bool_like(value: object, default: bool) -> bool:
    if value is None:
        return default
    if isinstance(value, bool):
        return value
    return str(value).strip().lower() in ("1", "true", "yes", "on")


def _kernel_policy(config: object | None = None) -> dict:
    if isinstance(config, dict):
        nested = config.get("kernel_policy")
        return nested if isinstance(nested, dict) else config
    policy = getattr(config, "kernel_policy", None)
    return policy if isinstance(policy, dict) else {}


def _kernel_policy_value(config: object | None, name: str, default: object = None) -> object:
    policy = _kernel_policy(config)
    return policy[name] if name in policy else default


def _scope_policy_value(value: object, default: str) -> str:
    scope = str(value or default).strip().lower()
    return scope if scope in ("all", "attention_only", "off") else default


def awq_fused_gemm_enabled(config: object | None = None) -> bool:
    """``awq_fused_gemm`` (default on): the fused dequant-GEMM is the primary path."""
    return _bool_like(_kernel_policy_value(config, "awq_fused_gemm", True), True)


def awq_fused_gemm_force_enabled(config: object | None = None) -> bool:
    """``awq_fused_gemm_force`` (default off): fused whatever the scope."""
    return _bool_like(_kernel_policy_value(config, "awq_fused_gemm_force", False), False)


def awq_decode_gemv_enabled(config: object | None = None) -> bool:
    return _bool_like(_kernel_policy_value(config, "awq_decode_gemv", False), False)


def awq_rows_exact_msmall_enabled(config: object | None = None) -> bool:
    """Policy key ``awq_rows_exact_msmall`` (``tensor.py:401-405``), default off: M = 2 / 4 keep
    the per-row M = 1 arithmetic."""
    return _bool_like(_kernel_policy_value(config, "awq_rows_exact_msmall", False), False)


def awq_group32_interleaved_down_proj_enabled(config: object | None = None) -> bool:
    return _bool_like(_kernel_policy_value(config, "awq_group32_interleaved_down_proj", False), False)


def gemma4_dense_down_proj_enabled(config: object | None = None) -> bool:
    return _bool_like(_kernel_policy_value(config, "gemma4_dense_down_proj", False), False)


def gemma4_dense_mlp_enabled(config: object | None = None) -> bool:
    return _bool_like(_kernel_policy_value(config, "gemma4_dense_mlp", False), False)


def awq_dense_fallback_cache_enabled(config: object | None = None) -> bool:
    return _bool_like(_kernel_policy_value(config, "awq_dense_fallback_cache", True), True)


def awq_cache_scope(config: object | None = None) -> str:
    return _scope_policy_value(_kernel_policy_value(config, "awq_cache_scope", "all"), "all")


def awq_fused_scope(config: object | None = None, profile_hint: str = "") -> str:
    """``awq_fused_scope`` when set; otherwise ``all`` for the profiled models
    (``qwen35_9b_awq``, ``gemma4_31b_q4``) and ``attention_only`` for the rest
    (``tensor.py:437-443``)."""
    raw = _kernel_policy_value(config, "awq_fused_scope", None)
    if raw is not None:
        return _scope_policy_value(raw, "all")
    if profile_hint in ("qwen35_9b_awq", "gemma4_31b_q4"):
        return "all"
    return "attention_only"


def _is_attention_like_prefix(prefix: str) -> bool:
    if not prefix:
        return False
    markers = (".self_attn.", ".linear_attn.", ".attn.", ".q_proj", ".k_proj", ".v_proj", ".o_proj")
    return any(m in prefix for m in markers)


def resolve_awq_execution_policy(prefix: str, x: torch.Tensor, profile_hint: str = "", *,
                                 config: object | None = None) -> AWQExecutionPolicy:
    cache_scope = awq_cache_scope(config)
    fused_scope = awq_fused_scope(config, profile_hint)
    allow_dense_cache = awq_dense_fallback_cache_enabled(config)
    if cache_scope == "off" or (cache_scope == "attention_only" and not _is_attention_like_prefix(prefix)):
        allow_dense_cache = False
    return AWQExecutionPolicy(prefer_fused=awq_fused_gemm_enabled(config), allow_dense_cache=allow_dense_cache,
                              cache_scope=cache_scope, fused_scope=fused_scope)


def should_allow_dense_cache(prefix: str, policy: AWQExecutionPolicy) -> bool:
    if not policy.allow_dense_cache:
        return False
    if policy.cache_scope == "attention_only":
        return _is_attention_like_prefix(prefix)
    return True


def should_allow_awq_fused(prefix: str, policy: AWQExecutionPolicy) -> tuple[bool, str]:
    if policy.fused_scope == "off":
        return False, "fused_scope_off"
    if policy.fused_scope == "attention_only" and not _is_attention_like_prefix(prefix):
        return False, "fused_scope_attention_only_non_attn"
    return True, "scope_ok"


def _capability(x, qweight, scales, qzeros, group_size, layout: str, symmetric: bool) -> tuple[bool, str]:
    """The reference's capability checks (``awq_triton.py:7-61``), K read per the weight's layout."""
    if symmetric:
        return _AT.packed_int4_fused_capability_check(x, qweight, scales, int(group_size), layout=layout)
    return _AT.awq_fused_capability_check(x, qweight, scales, qzeros, int(group_size), layout=layout)


def should_use_awq_fused_path(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
                              qzeros: torch.Tensor | None, group_size: int, prefix: str,
                              policy: AWQExecutionPolicy | None = None, *, config: object | None = None,
                              profile_hint: str = "", layout: str = "ref") -> tuple[bool, str]:
    """Force, then scope, then ``awq_fused_gemm``, then the capability check
    (``tensor.py:638-673``)."""
    resolved = policy or resolve_awq_execution_policy(prefix, x, profile_hint, config=config)
    if awq_fused_gemm_force_enabled(config):
        return True, "force_on"
    allow, reason = should_allow_awq_fused(prefix, resolved)
    if not allow:
        return False, reason
    if not resolved.prefer_fused:
        return False, "fused_disabled"
    try:
        return _capability(x, qweight, scales, qzeros, group_size, layout, False)
    except Exception as exc:
        return False, f"fused_capability_check_error:{type(exc).__name__}"


def _should_use_high_fidelity_awq(prefix: str, force_high_fidelity: bool = False) -> bool:
    if force_high_fidelity or _HIGH_FIDELITY_ALL:
        return True
    if not _HIGH_FIDELITY_PREFIX_MATCH or not prefix:
        return False
    return any(token in prefix for token in _HIGH_FIDELITY_PREFIXES)


def _is_gemma4_mlp_down_proj(prefix: str, profile_hint: str) -> bool:
    return profile_hint == "gemma4_31b_q4" and ".mlp.down_proj" in str(prefix)


def _is_gemma4_mlp_proj(prefix: str, profile_hint: str) -> bool:
    return profile_hint == "gemma4_31b_q4" and ".mlp." in str(prefix)


def _gemma4_down_proj_shape(x, qweight, group_size, layout) -> tuple[int, int, int] | None:
    if int(group_size) != 32 or x.dim() < 2:
        return None
    n = int(qweight.shape[0]) if layout == "ref" else int(qweight.shape[1]) * 8
    return int(x.reshape(-1, x.shape[-1]).shape[0]), n, int(x.shape[-1])


def _should_try_gemma4_down_proj(prefix, profile_hint, x, qweight, scales, group_size, layout,
                                 config) -> bool:
    """The Gemma4-31B MLP down projection's two decode routes (``tensor.py:495-540``): the
    interleaved group-32 GEMV (``awq_group32_interleaved_down_proj``, M = 1) and the fused GEMM
    with ``gemma4_dense_down_proj`` and ``awq_decode_gemv`` (M >= 1), both at N = 5376,
    K = 21504.  Here both run the fused HIP GEMM (the decode kernels read the weight in their
    own layout, so the reference's interleaved pack has no counterpart)."""
    if not _is_gemma4_mlp_down_proj(prefix, profile_hint):
        return False
    shape = _gemma4_down_proj_shape(x, qweight, group_size, layout)
    if shape is None or shape[1:] != (5376, 21504):
        return False
    if awq_group32_interleaved_down_proj_enabled(config) and shape[0] == 1 and \
            scales.dtype in (torch.float16, torch.bfloat16):
        return True
    return gemma4_dense_down_proj_enabled(config) and awq_decode_gemv_enabled(config) and shape[0] >= 1


def _apply_linear_with_cached_weight(x, w, bias):
    _stat("cached_mode_dense")
    return F.linear(x, w if w.dtype == x.dtype else w.to(x.dtype), bias)


class QuantizedLinearWeight(nn.Module, ABC):
    def __init__(self):
        super().__init__()
        self.weight_id = id(self)

    @abstractmethod
    def matmul(self, x: torch.Tensor, bias: torch.Tensor | None = None, *,
               config: object | None = None) -> torch.Tensor:
        ...


class AWQWeight(QuantizedLinearWeight):
    """Zero-point AWQ weight.  ``layout="ref"`` (default) takes the reference runtime
    tensors ``qweight [N, K/8]``, ``scales [N, K/G]``, ``qzeros [N, K/G/8]``;
    ``layout="autoawq"`` takes AutoAWQ checkpoint tensors ``[K, N/8]``, ``[K/G, N]``,
    ``[K/G, N/8]`` as they are."""

    _symmetric = False

    def __init__(self, qweight, scales, qzeros, group_size=128, prefix: str = "",
                 high_fidelity: bool = False, profile_hint: str = "", layout: str = "ref"):
        super().__init__()
        self.qweight = nn.Parameter(qweight, requires_grad=False)
        self.scales = nn.Parameter(scales, requires_grad=False)
        self.qzeros = nn.Parameter(qzeros, requires_grad=False) if qzeros is not None else None
        self.group_size = int(group_size)
        self.prefix = prefix
        self.high_fidelity = high_fidelity
        self.profile_hint = profile_hint
        self.layout = layout

    # -- fused path -------------------------------------------------------------
    def _fused(self, x2, bias, config):
        if self._symmetric:
            return _AFG.packed_int4_symmetric_fused_gemm_safe(
                x2, self.qweight, self.scales, self.group_size, bias=bias, config=config, layout=self.layout)
        return _AFG.awq_fused_gemm_safe(x2, self.qweight, self.scales, self.qzeros, self.group_size,
                                        bias=bias, config=config, layout=self.layout)

    def _try_fused(self, x, bias, config):
        """One fused call with the reference's counters; the output, or None when refused."""
        _stat("awq_fused_attempt")
        _prefix_stat(self.prefix, "fused_attempt")
        try:
            out, used, reason = self._fused(x.reshape(-1, x.shape[-1]).contiguous(), bias, config)
        except Exception:
            _prefix_stat(self.prefix, "fused_runtime_exception")
            return None
        if used:
            _stat("awq_fused_success")
            _prefix_stat(self.prefix, "fused_success")
            return out.view(*x.shape[:-1], out.shape[-1])
        _prefix_stat(self.prefix, "fused_runtime_fallback")
        if reason:
            _prefix_stat(self.prefix, f"reason:{reason}")
        return None

    # -- dense fallback ---------------------------------------------------------
    def dense_weight(self, dtype: torch.dtype = torch.float16) -> torch.Tensor:
        """[N, K] dense weight (HIP dequant kernel), transposed for the KN layouts."""
        w = ops.dequant(self.qweight, self.scales, self.qzeros, self.group_size,
                        layout=self.layout, out_dtype=torch.float16)
        if self.layout != "ref":
            w = w.t().contiguous()
        return w if dtype == torch.float16 else w.to(dtype)

    def _slow_matmul_dequant(self, x, bias):
        """The dense path (``tensor.py:1124-1147``): the cached dense weight, or one built by the
        HIP dequant kernel and put in the LRU."""
        w = _GLOBAL_WEIGHT_CACHE.get(self.weight_id)
        if w is not None:
            _stat("awq_cache_hits")
            _prefix_stat(self.prefix, "cache_hit")
            return _apply_linear_with_cached_weight(x, w, bias)
        w = self.dense_weight()
        _ensure_dense_budget()
        _GLOBAL_WEIGHT_CACHE.put(self.weight_id, w)
        _stat("awq_cache_misses")
        _stat("awq_dense_builds")
        _prefix_stat(self.prefix, "cache_miss")
        _prefix_stat(self.prefix, "dense_build")
        return F.linear(x, w if w.dtype == x.dtype else w.to(x.dtype), bias)

    def matmul(self, x, bias=None, *, config: object | None = None):
        """``tensor.py:1008-1122``: the frozen decision (fused, falling back to the dense path
        on a refusal) or, on the first call, high fidelity -> dense, else the execution policy
        (force, scope, ``awq_fused_gemm``, capability) decides, is frozen, and the call re-enters
        (so the first call counts twice in ``matmul_calls``, as in the reference)."""
        _stat("awq_matmul_calls")
        _prefix_stat(self.prefix, "matmul_calls")
        decision = getattr(self, "_cached_fused_decision", None)
        if decision is not None:
            if decision:
                out = self._try_fused(x, bias, config)
                if out is not None:
                    return out
            return self._slow_matmul_dequant(x, bias)
        if _should_use_high_fidelity_awq(self.prefix, self.high_fidelity):
            self._cached_fused_decision = False
            _prefix_stat(self.prefix, "high_fidelity_forced")
            return self._slow_matmul_dequant(x, bias)
        policy = resolve_awq_execution_policy(self.prefix, x, self.profile_hint, config=config)
        use_fused, reason = should_use_awq_fused_path(
            x, self.qweight, self.scales, self.qzeros, self.group_size, self.prefix, policy, config=config,
            profile_hint=self.profile_hint, layout=self.layout)
        if use_fused:
            _prefix_stat(self.prefix, "decision_fused")
        else:
            _prefix_stat(self.prefix, "decision_dense")
            if reason:
                _prefix_stat(self.prefix, f"reason:{reason}")
        self._cached_fused_decision = bool(use_fused)
        return self.matmul(x, bias, config=config)


class PackedInt4Weight(AWQWeight):
    """Zero-point-free int4 weight, ``W = (q - 8) * s`` (``tensor.py:1150-1451``)."""

    _symmetric = True

    def __init__(self, qweight, scales, group_size=128, original_shape=None, prefix: str = "",
                 high_fidelity: bool = False, profile_hint: str = "", layout: str = "ref"):
        super().__init__(qweight.to(torch.int32) if qweight.dtype != torch.int32 else qweight,
                         scales, None, group_size, prefix, high_fidelity, profile_hint, layout)
        self.original_shape = original_shape

    def matmul(self, x, bias=None, *, config: object | None = None):
        """The reference's order (``tensor.py:1170-1451``): row-exact M = 2 / 4 when asked, the
        Gemma4 down-projection routes, the Gemma4 dense-MLP switches, the frozen decision, then
        on the first call high fidelity, force, scope and the capability check."""
        _stat("awq_matmul_calls")
        _prefix_stat(self.prefix, "matmul_calls")
        x2 = x.reshape(-1, x.shape[-1])
        if awq_rows_exact_msmall_enabled(config) and int(x2.shape[0]) in (2, 4):
            try:
                out, used, reason = _AFG.packed_int4_symmetric_group32_rows_exact_msmall_safe(
                    x2.contiguous(), self.qweight, self.scales, int(self.group_size), bias=bias)
                if used:
                    _stat("awq_rows_exact_msmall_success")
                    _prefix_stat(self.prefix, "rows_exact_msmall_success")
                    return out.view(*x.shape[:-1], out.shape[-1])
                _prefix_stat(self.prefix, f"rows_exact_msmall_fallback:{reason}")
            except Exception as exc:
                _prefix_stat(self.prefix, f"rows_exact_msmall_exception:{type(exc).__name__}")
            # a refused row-exact call never falls to the generic batched GEMM: one M = 1 call per row
            rows = [self.matmul(x2[r:r + 1], bias, config=config) for r in range(int(x2.shape[0]))]
            return torch.cat(rows, dim=0).view(*x.shape[:-1], rows[0].shape[-1])

        if _should_try_gemma4_down_proj(self.prefix, self.profile_hint, x, self.qweight, self.scales,
                                        self.group_size, self.layout, config):
            out = self._try_fused(x, bias, config)
            if out is not None:
                _prefix_stat(self.prefix, "decision_fused_gemma4_down_proj")
                return out
        if (gemma4_dense_mlp_enabled(config) and _is_gemma4_mlp_proj(self.prefix, self.profile_hint)) or \
                (gemma4_dense_down_proj_enabled(config) and _is_gemma4_mlp_down_proj(self.prefix, self.profile_hint)):
            self._cached_fused_decision = False
            _prefix_stat(self.prefix, "decision_dense_gemma4_mlp")
            return self._slow_matmul_dequant(x, bias)

        decision = getattr(self, "_cached_fused_decision", None)
        if decision is True:
            out = self._try_fused(x, bias, config)
            if out is not None:
                return out
            self._cached_fused_decision = False  # a refusal freezes the dense path
            return self._slow_matmul_dequant(x, bias)
        if decision is False:
            _prefix_stat(self.prefix, "decision_dense_cached")
            return self._slow_matmul_dequant(x, bias)
        if _should_use_high_fidelity_awq(self.prefix, self.high_fidelity):
            self._cached_fused_decision = False
            _prefix_stat(self.prefix, "high_fidelity_forced")
            return self._slow_matmul_dequant(x, bias)
        if awq_fused_gemm_force_enabled(config):
            self._cached_fused_decision = True
            _prefix_stat(self.prefix, "decision_fused_forced")
            return self.matmul(x, bias, config=config)
        policy = resolve_awq_execution_policy(self.prefix, x, self.profile_hint, config=config)
        allow, reason = should_allow_awq_fused(self.prefix, policy)
        if not allow:
            self._cached_fused_decision = False
            _prefix_stat(self.prefix, "decision_dense")
            _prefix_stat(self.prefix, f"reason:{reason}")
            return self._slow_matmul_dequant(x, bias)
        use_fused = False
        if policy.prefer_fused:
            try:
                use_fused, _ = _capability(x, self.qweight, self.scales, None, self.group_size, self.layout, True)
            except Exception:
                _prefix_stat(self.prefix, "capability_check_exception")
        self._cached_fused_decision = bool(use_fused)
        if use_fused:
            _prefix_stat(self.prefix, "decision_fused")
            return self.matmul(x, bias, config=config)
        _prefix_stat(self.prefix, "decision_dense")
        return self._slow_matmul_dequant(x, bias)

    def dense_weight(self, dtype: torch.dtype = torch.float16) -> torch.Tensor:
        w = super().dense_weight(dtype)
        if self.original_shape is not None:
            w = w[: self.original_shape[0], : self.original_shape[1]].contiguous()
        return w
