"""Drop-in for the AWQ entry points of ``vllm/kernels/triton/awq_fused_gemm.py``:
``awq_fused_gemm``, ``awq_fused_gemm_safe``, ``packed_int4_symmetric_fused_gemm`` and
``packed_int4_symmetric_fused_gemm_safe`` keep the reference's arguments, validation,
reason strings and split-K knob; the launch goes to the gfx950 HIP kernels.

Differences, all deliberate:
  * split-K partials are reduced in fp32 in a fixed order (the reference rounds each
    partial to fp16 and ``atomic_add``s it, ``awq_fused_gemm.py:1857-1866``), and bias is
    applied once whatever the split (the reference drops it when split_k > 1, ``1867-1880``);
  * with ``split_k`` unset ("auto") the MI355X planner picks the K partition for a full
    chip; the reference's auto heuristic (``awq_fused_gemm.py:420-501``) is tuned for a
    16-24-program grid on gfx1151 and is not reproduced;
  * bf16 activations always use bf16 MFMA operands with weights rounded once to bf16
    (the reference may narrow bf16 activations to fp16 for small shapes, ``113-139``);
  * ``layout=`` selects the packed layout ("ref" = reference runtime layout, the default;
    "autoawq" = AutoAWQ [K, N/8] checkpoints).
"""
from __future__ import annotations

from typing import Any

import torch

from . import ops

_AWQ_FUSED_TUNING: dict[str, str] = {}
_AWQ_FUSED_TUNING_LOCKED = False


def set_awq_fused_tuning_config(values: dict[str, object] | None, *, locked: bool = False) -> None:
    """Install the tuning snapshot (``awq_fused_gemm.py:15-31``); only the split-K key is read."""
    global _AWQ_FUSED_TUNING, _AWQ_FUSED_TUNING_LOCKED
    _AWQ_FUSED_TUNING = {str(k): str(v) for k, v in (values or {}).items() if v is not None}
    _AWQ_FUSED_TUNING_LOCKED = bool(locked)


def _kernel_policy(config: Any | None = None, policy: dict | None = None) -> dict:
    if isinstance(policy, dict):
        return policy
    if isinstance(config, dict):
        nested = config.get("kernel_policy")
        return nested if isinstance(nested, dict) else config
    kp = getattr(config, "kernel_policy", None)
    return kp if isinstance(kp, dict) else {}


def _parse_split(raw) -> int | None:
    if raw is None:
        return None
    s = str(raw).strip().lower()
    if s in ("", "auto"):
        return None
    try:
        return max(1, int(s))
    except ValueError:
        return 1


def _select_split_k(m: int, n: int, k: int, *, config: Any | None = None,
                    policy: dict | None = None) -> int:
    """Split-K knob with the reference's precedence (``awq_fused_gemm.py:420-469``):
    tool override, then ``kernel_policy["awq_fused_gemm_split_k"]``, then the tuning
    snapshot.  Returns 0 for "auto" (the library plans the partition)."""
    for raw in (_AWQ_FUSED_TUNING.get("FASTINFERENCE_AWQ_FUSED_GEMM_SPLIT_K"),
                _kernel_policy(config, policy).get("awq_fused_gemm_split_k")):
        v = _parse_split(raw)
        if v is not None:
            return v
    return 0


def _validate_bias(bias, n, a):
    if bias.dim() != 1 or int(bias.shape[0]) != n:
        raise ValueError(f"awq_fused_gemm: bias must be 1D of size N={n}, got {tuple(bias.shape)}")
    if bias.device != a.device:
        raise ValueError("awq_fused_gemm: bias must be on the same device as activations")
    if bias.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"awq_fused_gemm: unsupported bias dtype {bias.dtype}")
    return bias.contiguous().reshape(n)


def awq_fused_gemm(a, qweight, scales, qzeros, group_size, out=None, bias=None, *,
                   config: Any | None = None, policy: dict | None = None, layout: str = "ref"):
    """``C[M, N] = a[M, K] @ dequant(qweight)^T (+ bias)`` (``awq_fused_gemm.py:2395-2552``)."""
    M, K = a.shape
    _, N = ops.gemm_dims(qweight, layout)
    if bias is not None:
        bias = _validate_bias(bias, N, a)
    split_k = _select_split_k(M, N, K, config=config, policy=policy)
    return ops.gemm(a, qweight, scales, qzeros, int(group_size), bias=bias, split_k=split_k,
                    layout=layout, out=out)


def packed_int4_symmetric_fused_gemm(a, qweight, scales, group_size, out=None, bias=None, *,
                                     config: Any | None = None, policy: dict | None = None,
                                     layout: str = "ref"):
    """Symmetric mode ``(q - 8) * s`` (``awq_fused_gemm.py:2555-2922``)."""
    M, K = a.shape
    _, N = ops.gemm_dims(qweight, layout)
    if bias is not None:
        bias = _validate_bias(bias, N, a)
    split_k = _select_split_k(M, N, K, config=config, policy=policy)
    return ops.gemm(a, qweight.to(torch.int32) if qweight.dtype != torch.int32 else qweight,
                    scales, None, int(group_size), bias=bias, split_k=split_k, layout=layout, out=out)


def _common_checks(a, qweight, scales, group_size, bias, layout):
    if a.dim() != 2:
        return "input_not_2d"
    if qweight.dim() != 2:
        return "qweight_not_2d"
    if scales.dim() != 2:
        return "scales_not_2d"
    return None


def _shape_checks(a, qweight, scales, group_size, bias, layout, extra_devices=()):
    k = int(a.shape[1])
    kw, n = ops.gemm_dims(qweight, layout)
    if k != kw:
        return "k_mismatch"
    if group_size <= 0 or k % int(group_size) != 0:
        return "group_mismatch"
    if a.device != qweight.device or a.device != scales.device or any(
            d is not None and a.device != d.device for d in extra_devices):
        return "device_mismatch"
    if a.dtype not in (torch.float16, torch.bfloat16):
        return f"unsupported_dtype_{str(a.dtype)}"
    if bias is not None:
        if bias.dim() != 1 or int(bias.numel()) != n:
            return "bias_bad_shape"
        if bias.device != a.device:
            return "bias_device_mismatch"
        if bias.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            return f"unsupported_bias_dtype_{str(bias.dtype)}"
    return None


def awq_fused_gemm_safe(a, qweight, scales, qzeros, group_size, out=None, bias=None, *,
                        config: Any | None = None, policy: dict | None = None,
                        layout: str = "ref") -> tuple[torch.Tensor, bool, str]:
    """Never raises; returns ``(C, True, "ok")`` or ``(a, False, reason)`` with the
    reference's reason strings (``awq_fused_gemm.py:3713-3775``)."""
    r = _common_checks(a, qweight, scales, group_size, bias, layout)
    if r:
        return a, False, r
    if qzeros is None or qzeros.dim() != 2:
        return a, False, "qzeros_bad"
    r = _shape_checks(a, qweight, scales, group_size, bias, layout, (qzeros,))
    if r:
        return a, False, r
    m = int(a.shape[0])
    n = ops.gemm_dims(qweight, layout)[1]
    try:
        c = awq_fused_gemm(a.contiguous(), qweight.contiguous(), scales.contiguous(),
                           qzeros.contiguous(), group_size=group_size, out=out,
                           bias=bias.contiguous() if bias is not None else None,
                           config=config, policy=policy, layout=layout)
        if c.shape != (m, n):
            return c, False, "bad_output_shape"
        return c, True, "ok"
    except Exception:
        return a, False, "kernel_exception"


def packed_int4_symmetric_fused_gemm_safe(a, qweight, scales, group_size, out=None, bias=None, *,
                                          config: Any | None = None, policy: dict | None = None,
                                          layout: str = "ref") -> tuple[torch.Tensor, bool, str]:
    """``awq_fused_gemm.py:3778-3831``."""
    r = _common_checks(a, qweight, scales, group_size, bias, layout)
    if r:
        return a, False, r
    r = _shape_checks(a, qweight, scales, group_size, bias, layout)
    if r:
        return a, False, r
    m = int(a.shape[0])
    n = ops.gemm_dims(qweight, layout)[1]
    try:
        c = packed_int4_symmetric_fused_gemm(
            a.contiguous(), qweight.contiguous(), scales.contiguous(), group_size=group_size,
            out=out, bias=bias.contiguous() if bias is not None else None, config=config,
            policy=policy, layout=layout)
        if c.shape != (m, n):
            return c, False, "bad_output_shape"
        return c, True, "ok"
    except Exception:
        return a, False, "kernel_exception"
