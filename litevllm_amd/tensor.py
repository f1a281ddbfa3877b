"""Drop-in for the AWQ weight objects of
``vllm/model_executor/layers/quantization/tensor.py``: ``QuantizedLinearWeight``,
``AWQWeight`` and ``PackedInt4Weight`` keep the ``matmul(x, bias=None, *, config=None)``
protocol (``tensor.py:946-959``), the frozen first-call fused/dense decision
(``tensor.py:1094-1122``), the dense-weight LRU fallback (``tensor.py:1085-1092,
1124-1147``) and the runtime counters (``tensor.py:226-243``).

Both paths run on the GPU: the fused path calls the HIP GEMM; the dense fallback
dequantizes with the HIP dequant kernel and multiplies with ``F.linear`` -- exactly the
reference's fallback structure.  Neither has a CPU branch.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from collections import OrderedDict, defaultdict
from typing import Any

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .awq_fused_gemm import (awq_fused_gemm_safe, packed_int4_symmetric_fused_gemm_safe,
                             packed_int4_symmetric_group32_rows_exact_msmall_safe)

_STATS: dict[str, int] = defaultdict(int)
_PREFIX_STATS: dict[str, dict[str, int]] = defaultdict(lambda: defaultdict(int))


def _stat(key: str, prefix: str = "", delta: int = 1) -> None:
    _STATS[key] += delta
    if prefix:
        _PREFIX_STATS[prefix][key] += delta


def get_awq_runtime_stats() -> dict[str, int]:
    return dict(_STATS)


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

    def clear(self) -> None:
        self._d.clear()
        self.current_bytes = 0


_GLOBAL_WEIGHT_CACHE = LRUWeightCache(max_size=256, max_bytes=14 << 30)


def clear_global_weight_cache() -> None:
    _GLOBAL_WEIGHT_CACHE.clear()


def _kernel_policy_value(config: Any | None, name: str, default=None):
    kp = config.get("kernel_policy", config) if isinstance(config, dict) else getattr(config, "kernel_policy", None)
    if isinstance(kp, dict) and name in kp:
        return kp[name]
    return default


def _truthy(v) -> bool:
    return v if isinstance(v, bool) else str(v).strip().lower() in ("1", "true", "yes", "on")


def awq_rows_exact_msmall_enabled(config: object | None = None) -> bool:
    """Policy key ``awq_rows_exact_msmall`` (``tensor.py:401-405``), default off: M = 2 / 4 keep
    the per-row M = 1 arithmetic."""
    return _truthy(_kernel_policy_value(config, "awq_rows_exact_msmall", False))


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
            return packed_int4_symmetric_fused_gemm_safe(
                x2, self.qweight, self.scales, self.group_size, bias=bias, config=config,
                layout=self.layout)
        return awq_fused_gemm_safe(x2, self.qweight, self.scales, self.qzeros, self.group_size,
                                   bias=bias, config=config, layout=self.layout)

    # -- dense fallback ---------------------------------------------------------
    def dense_weight(self, dtype: torch.dtype = torch.float16) -> torch.Tensor:
        """[N, K] dense weight (HIP dequant kernel), transposed for the KN layouts."""
        w = ops.dequant(self.qweight, self.scales, self.qzeros, self.group_size,
                        layout=self.layout, out_dtype=torch.float16)
        if self.layout != "ref":
            w = w.t().contiguous()
        return w if dtype == torch.float16 else w.to(dtype)

    def _slow_matmul_dequant(self, x, bias):
        w = _GLOBAL_WEIGHT_CACHE.get(self.weight_id)
        if w is not None:
            _stat("awq_cache_hits", self.prefix)
        else:
            w = self.dense_weight()
            _GLOBAL_WEIGHT_CACHE.put(self.weight_id, w)
            _stat("awq_cache_misses", self.prefix)
            _stat("awq_dense_builds", self.prefix)
        return F.linear(x, w if w.dtype == x.dtype else w.to(x.dtype), bias)

    def matmul(self, x, bias=None, *, config: object | None = None):
        _stat("awq_matmul_calls", self.prefix)
        decision = getattr(self, "_cached_fused_decision", None)
        if decision is None:
            # first call: freeze the decision for the lifetime of the object
            enabled = _truthy(_kernel_policy_value(config, "awq_fused_gemm", True))
            decision = bool(enabled and not self.high_fidelity and x.is_cuda)
            self._cached_fused_decision = decision
        if decision:
            _stat("awq_fused_attempt", self.prefix)
            x2 = x.reshape(-1, x.shape[-1]).contiguous()
            out, used, reason = self._fused(x2, bias, config)
            if used:
                _stat("awq_fused_success", self.prefix)
                return out.view(*x.shape[:-1], out.shape[-1])
            _stat(f"reason:{reason}", self.prefix)
            _stat("fused_runtime_fallback", self.prefix)
        return self._slow_matmul_dequant(x, bias)


class PackedInt4Weight(AWQWeight):
    """Zero-point-free int4 weight, ``W = (q - 8) * s`` (``tensor.py:1150-1451``)."""

    _symmetric = True

    def __init__(self, qweight, scales, group_size=128, original_shape=None, prefix: str = "",
                 high_fidelity: bool = False, profile_hint: str = "", layout: str = "ref"):
        super().__init__(qweight.to(torch.int32) if qweight.dtype != torch.int32 else qweight,
                         scales, None, group_size, prefix, high_fidelity, profile_hint, layout)
        self.original_shape = original_shape

    def matmul(self, x, bias=None, *, config: object | None = None):
        """With ``awq_rows_exact_msmall`` on and M in {2, 4}, the row-exact kernel path, or on its
        refusal one M = 1 call per row -- never the generic batched GEMM (``tensor.py:1200-1234``)."""
        x2 = x.reshape(-1, x.shape[-1])
        if awq_rows_exact_msmall_enabled(config) and int(x2.shape[0]) in (2, 4):
            try:
                out, used, reason = packed_int4_symmetric_group32_rows_exact_msmall_safe(
                    x2.contiguous(), self.qweight, self.scales, int(self.group_size), bias=bias)
                if used:
                    _stat("awq_rows_exact_msmall_success")
                    _stat("rows_exact_msmall_success", self.prefix)
                    return out.view(*x.shape[:-1], out.shape[-1])
                _stat(f"rows_exact_msmall_fallback:{reason}", self.prefix)
            except Exception as exc:
                _stat(f"rows_exact_msmall_exception:{type(exc).__name__}", self.prefix)
            rows = [self.matmul(x2[r:r + 1], bias, config=config) for r in range(int(x2.shape[0]))]
            return torch.cat(rows, dim=0).view(*x.shape[:-1], rows[0].shape[-1])
        return super().matmul(x, bias, config=config)

    def dense_weight(self, dtype: torch.dtype = torch.float16) -> torch.Tensor:
        w = super().dense_weight(dtype)
        if self.original_shape is not None:
            w = w[: self.original_shape[0], : self.original_shape[1]].contiguous()
        return w
