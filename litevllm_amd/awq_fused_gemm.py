"""Drop-in for the AWQ entry points of ``vllm/kernels/triton/awq_fused_gemm.py``:
``awq_fused_gemm``, ``awq_fused_gemm_safe``, ``packed_int4_symmetric_fused_gemm`` and
``packed_int4_symmetric_fused_gemm_safe`` keep the reference's arguments, validation,
reason strings and split-K knob; the launch goes to the gfx950 HIP kernels.  The M = 1
fused gate/up surfaces (``packed_int4_symmetric_fused_gate_up_m1``, its ``group32`` twin,
``..._m1_safe`` and the two policy switches) do the same for the gated MLP, and the fused QKV
surfaces (``packed_int4_symmetric_fused_qkv_m1/_m2(_safe)``, ``awq_decode_gemv_enabled``) for
the attention projections.

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


def _parse_forced(raw) -> int:
    """A forced split-K value: an integer clamped to >= 1, anything unparsable (the empty
    string included) 1 -- ``int(raw)`` with the reference's ``ValueError`` fallback
    (``awq_fused_gemm.py:436-441``)."""
    try:
        return max(1, int(str(raw).strip().lower()))
    except ValueError:
        return 1


def _select_split_k(m: int, n: int, k: int, *, config: Any | None = None,
                    policy: dict | None = None) -> int:
    """Split-K knob with the reference's precedence (``awq_fused_gemm.py:420-469``):
      * the tool override ``FASTINFERENCE_AWQ_FUSED_GEMM_SPLIT_K`` of the tuning snapshot, when
        the key is present at all (an empty or unparsable value forces 1, as ``int()``'s
        ``ValueError`` does there);
      * ``kernel_policy["awq_fused_gemm_split_k"]`` unless it is ``""`` or ``"auto"``;
      * otherwise "auto".  (The reference's later snapshot lookup, ``456-462``, can only see a
        key the tool override has already taken, so it never decides.)
    Returns 0 for "auto": the library plans the partition for the MI355X (the reference's
    auto rule, ``470-501``, sizes a 16-24-program gfx1151 grid and is not reproduced)."""
    if "FASTINFERENCE_AWQ_FUSED_GEMM_SPLIT_K" in _AWQ_FUSED_TUNING:
        return _parse_forced(_AWQ_FUSED_TUNING["FASTINFERENCE_AWQ_FUSED_GEMM_SPLIT_K"])
    kp = _kernel_policy(config, policy)
    if "awq_fused_gemm_split_k" in kp:
        # a present None reaches the reference's last lookup as the string "none": forced 1
        raw = str(kp["awq_fused_gemm_split_k"]).strip().lower()
        if raw not in ("", "auto"):
            return _parse_forced(raw)
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
    if out is not None:
        r = ops.out_problem(out, m, n, a)
        if r:  # checked before the launch: the kernels would write M x N values into it
            return a, False, r
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
    if out is not None:
        r = ops.out_problem(out, m, n, a)
        if r:
            return a, False, r
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


def packed_int4_symmetric_group32_rows_exact_msmall_safe(a, qweight, scales, group_size, out=None, bias=None
                                                         ) -> tuple[torch.Tensor, bool, str]:
    """Row-exact M = 2 / 4 symmetric group-32 GEMM (``awq_fused_gemm.py:2925-2998``): every row
    equals, bit for bit, the M = 1 call on that row alone (``ops.gemm_rows_exact``: each row
    runs the M = 1 plan and kernel).  Same checks, order and reasons as the reference; never
    raises.  Reference layout (``qweight [N, K/8]``, ``scales [N, K/32]``)."""
    if a.dim() != 2 or int(a.shape[0]) not in (2, 4):
        return a, False, "input_not_m2_or_m4_2d"
    if qweight.dim() != 2 or scales.dim() != 2:
        return a, False, "weight_or_scales_not_2d"
    m, k = int(a.shape[0]), int(a.shape[1])
    n = int(qweight.shape[0])
    if int(group_size) != 32 or k % 32 != 0:
        return a, False, "unsupported_group_layout"
    if k != int(qweight.shape[1]) * 8:
        return a, False, "k_mismatch"
    if tuple(scales.shape) != (n, k // 32):
        return a, False, "scales_shape_mismatch"
    if a.device != qweight.device or a.device != scales.device or a.dtype not in (torch.float16, torch.bfloat16):
        return a, False, "tensor_device_or_dtype"
    if bias is not None and (bias.dim() != 1 or int(bias.numel()) != n or bias.device != a.device
                             or bias.dtype not in (torch.float16, torch.bfloat16, torch.float32)):
        return a, False, "bias_layout_or_dtype"
    if not (a.is_contiguous() and qweight.is_contiguous() and scales.is_contiguous()):
        return a, False, "noncontiguous_input"
    if out is not None and (tuple(out.shape) != (m, n) or out.device != a.device or out.dtype != a.dtype
                            or out.stride(1) != 1):
        return a, False, "bad_output"
    try:
        qw = qweight if qweight.dtype == torch.int32 else qweight.to(torch.int32)
        c = ops.gemm_rows_exact(a, qw, scales, None, 32, bias=bias, layout="ref", out=out)
        return c, True, "ok"
    except Exception:
        return a, False, "kernel_exception"


# ------------------------------------------------------------------ fused gate/up (M = 1)
def _truthy(value) -> bool:
    return str(value or "").strip().lower() in ("1", "true", "yes", "on")


def _policy_flag(config, policy, name: str) -> bool:
    raw = _kernel_policy(config, policy).get(name, False)
    return raw if isinstance(raw, bool) else _truthy(raw)


def awq_fused_gate_up_enabled(*, config: Any | None = None, policy: dict | None = None) -> bool:
    """Policy key ``awq_fused_gate_up``, default off (``awq_fused_gemm.py:513-519``)."""
    return _policy_flag(config, policy, "awq_fused_gate_up")


def awq_fused_gate_up_group32_enabled(*, config: Any | None = None, policy: dict | None = None) -> bool:
    """Policy key ``awq_fused_gate_up_group32``, default off (``awq_fused_gemm.py:522-528``)."""
    return _policy_flag(config, policy, "awq_fused_gate_up_group32")


def _gate_up_m1(name, a, gate_qweight, up_qweight, gate_scales, up_scales, group_size, activation, out):
    m, k = a.shape
    if m != 1:
        raise ValueError(f"{name}: requires M == 1")
    if int(group_size) != 32 or k % 32 != 0:
        raise ValueError(f"{name}: requires group_size=32 and K%32==0")
    if tuple(gate_qweight.shape) != tuple(up_qweight.shape):
        raise ValueError(f"{name}: qweight shape mismatch")
    if tuple(gate_scales.shape) != tuple(up_scales.shape):
        raise ValueError(f"{name}: scale shape mismatch")
    if int(gate_qweight.shape[1]) * 8 != k:
        raise ValueError(f"{name}: K mismatch")
    if out is not None and out.dtype != a.dtype:
        raise ValueError(f"{name}: out must have the input's dtype")
    as_i32 = lambda t: t if t.dtype == torch.int32 else t.to(torch.int32)
    return ops.gate_up_act(a, as_i32(gate_qweight), as_i32(up_qweight), gate_scales, up_scales,
                           int(group_size), activation=activation, layout="ref", out=out)


def packed_int4_symmetric_fused_gate_up_m1(a, gate_qweight, up_qweight, gate_scales, up_scales,
                                           group_size, *, activation: str = "silu", out=None,
                                           config: Any | None = None, policy: dict | None = None):
    """``out[0, n] = act(a . Wg[n]) * (a . Wu[n])`` for symmetric packed int4 (z = 8) weights
    in the reference layout [N, K/8] with scales [N, K/32] (``awq_fused_gemm.py:3009-3071``,
    kernel 1406-1506): one launch of the decode kernel with its gated epilogue over the cached
    interleaved pair; sums in fp32 over unrounded (q - 8) * s, one rounding at the end."""
    del config, policy
    return _gate_up_m1("packed_int4_symmetric_fused_gate_up_m1", a, gate_qweight, up_qweight,
                       gate_scales, up_scales, group_size, activation, out)


def packed_int4_symmetric_fused_gate_up_group32_m1(a, gate_qweight, up_qweight, gate_scales,
                                                   up_scales, group_size, *, activation: str = "silu",
                                                   out=None, config: Any | None = None,
                                                   policy: dict | None = None):
    """The reference's group-oriented twin (``awq_fused_gemm.py:3074-3120``) computes the same
    function; here both run the same kernel."""
    del config, policy
    m, k = a.shape
    if m != 1 or int(group_size) != 32 or k % 32 != 0:
        raise ValueError("group32 fused gate/up requires M=1 and aligned group32 K")
    if tuple(gate_qweight.shape) != tuple(up_qweight.shape):
        raise ValueError("group32 fused gate/up qweight shape mismatch")
    if tuple(gate_scales.shape) != tuple(up_scales.shape):
        raise ValueError("group32 fused gate/up scale shape mismatch")
    if int(gate_qweight.shape[1]) * 8 != k:
        raise ValueError("group32 fused gate/up K mismatch")
    return _gate_up_m1("group32 fused gate/up", a, gate_qweight, up_qweight, gate_scales, up_scales,
                       group_size, activation, out)


def packed_int4_symmetric_fused_gate_up_m1_safe(a, gate_qweight, up_qweight, gate_scales, up_scales,
                                                group_size, *, activation: str = "silu", out=None,
                                                config: Any | None = None, policy: dict | None = None
                                                ) -> tuple[torch.Tensor, bool, str]:
    """Never raises; ``(out, True, "ok")`` or ``(a, False, reason)`` with the reference's
    checks, order and reason strings (``awq_fused_gemm.py:3647-3710``)."""
    if not awq_fused_gate_up_enabled(config=config, policy=policy):
        return a, False, "disabled"
    if a.dim() != 2 or int(a.shape[0]) != 1:
        return a, False, "input_not_m1_2d"
    if gate_qweight.dim() != 2 or up_qweight.dim() != 2:
        return a, False, "qweight_not_2d"
    if gate_scales.dim() != 2 or up_scales.dim() != 2:
        return a, False, "scales_not_2d"
    if tuple(gate_qweight.shape) != tuple(up_qweight.shape):
        return a, False, "qweight_shape_mismatch"
    if tuple(gate_scales.shape) != tuple(up_scales.shape):
        return a, False, "scale_shape_mismatch"
    if a.dtype not in (torch.float16, torch.bfloat16):
        return a, False, f"unsupported_dtype_{str(a.dtype)}"
    if int(group_size) != 32:
        return a, False, "group_size_not_32"
    if int(a.shape[1]) != int(gate_qweight.shape[1]) * 8:
        return a, False, "k_mismatch"
    if int(a.shape[1]) % 32 != 0:
        return a, False, "k_not_group_aligned"
    dev = a.device
    if any(t.device != dev for t in (gate_qweight, up_qweight, gate_scales, up_scales)):
        return a, False, "device_mismatch"
    try:
        runner = (packed_int4_symmetric_fused_gate_up_group32_m1
                  if awq_fused_gate_up_group32_enabled(config=config, policy=policy)
                  else packed_int4_symmetric_fused_gate_up_m1)
        c = runner(a.contiguous(), gate_qweight.contiguous(), up_qweight.contiguous(),
                   gate_scales.contiguous(), up_scales.contiguous(), int(group_size),
                   activation=activation, out=out, config=config, policy=policy)
        if c.shape != (1, int(gate_qweight.shape[0])):
            return c, False, "bad_output_shape"
        return c, True, "ok"
    except Exception:
        return a, False, "kernel_exception"


# ------------------------------------------------------------------ fused QKV (M = 1, 2)
def awq_decode_gemv_enabled(*, config: Any | None = None, policy: dict | None = None) -> bool:
    """Policy key ``awq_decode_gemv``, default off (``awq_fused_gemm.py:503-509``)."""
    return _policy_flag(config, policy, "awq_decode_gemv")


def _concat_qkv(q_qweight, k_qweight, v_qweight, q_scales, k_scales, v_scales):
    """q | k | v along N in the reference layout, rows padded to a multiple of 8 with zero
    weights and zero scales (built once per weight triple and cached)."""
    qw = [q_qweight, k_qweight] + ([v_qweight] if v_qweight is not None else [])
    sc = [q_scales, k_scales] + ([v_scales] if v_scales is not None else [])
    qw = torch.cat([t.to(torch.int32) for t in qw], 0)
    sc = torch.cat(list(sc), 0)
    pad = (-int(qw.shape[0])) % 8
    if pad:
        qw = torch.cat([qw, qw.new_zeros((pad, qw.shape[1]))], 0)
        sc = torch.cat([sc, sc.new_zeros((pad, sc.shape[1]))], 0)
    return qw.contiguous(), sc.contiguous()


_QKV_CACHE = ops._DerivedCache("qkv_concat", _concat_qkv)


def _qkv(a, q_qweight, k_qweight, v_qweight, q_scales, k_scales, v_scales, group_size, out):
    has_v = v_qweight is not None and v_scales is not None
    if not has_v:
        v_qweight = v_scales = None
    total_n = int(q_qweight.shape[0]) + int(k_qweight.shape[0]) + (int(v_qweight.shape[0]) if has_v else 0)
    qw, sc = _QKV_CACHE.get(q_qweight, k_qweight, v_qweight, q_scales, k_scales, v_scales)
    m = int(a.shape[0])
    if out is None:
        out = torch.empty((m, total_n), device=a.device, dtype=a.dtype)
    if int(qw.shape[0]) == total_n and out.is_contiguous():
        return ops.gemm(a, qw, sc, None, int(group_size), layout="ref", out=out)
    y = ops.gemm(a, qw, sc, None, int(group_size), layout="ref")
    out.copy_(y[:, :total_n])
    return out


def packed_int4_symmetric_fused_qkv_m1(a, q_qweight, k_qweight, v_qweight, q_scales, k_scales, v_scales,
                                       group_size, *, out=None, config: Any | None = None,
                                       policy: dict | None = None):
    """``[q | k | v] = a @ W^T`` for symmetric packed int4 (z = 8) reference-layout projections
    in one launch (``awq_fused_gemm.py:3345-3423``; kernel ``1286-1402``): the three weights
    concatenated along N once (cached) and served by the decode kernels, unrounded
    ``(q - 8) * s`` weights summed in fp32, one rounding."""
    m, k = a.shape
    if m != 1:
        raise ValueError("packed_int4_symmetric_fused_qkv_m1: requires M == 1")
    if int(group_size) != 32 or k % 32 != 0:
        raise ValueError("packed_int4_symmetric_fused_qkv_m1: requires group_size=32 and K%32==0")
    del config, policy
    return _qkv(a, q_qweight, k_qweight, v_qweight, q_scales, k_scales, v_scales, group_size, out)


def packed_int4_symmetric_fused_qkv_m2(a, q_qweight, k_qweight, v_qweight, q_scales, k_scales, v_scales,
                                       group_size, *, config: Any | None = None, policy: dict | None = None):
    """The M = 2 form (``awq_fused_gemm.py:3426-3523``)."""
    if int(a.shape[0]) != 2:
        raise ValueError("packed_int4_symmetric_fused_qkv_m2: requires M == 2")
    del config, policy
    return _qkv(a, q_qweight, k_qweight, v_qweight, q_scales, k_scales, v_scales, group_size, None)


def packed_int4_symmetric_fused_qkv_m1_safe(a, q_qweight, k_qweight, v_qweight, q_scales, k_scales, v_scales,
                                            group_size, *, config: Any | None = None,
                                            policy: dict | None = None) -> tuple[torch.Tensor, bool, str]:
    """Never raises; the reference's checks, order and reasons (``awq_fused_gemm.py:3526-3589``)."""
    if not awq_decode_gemv_enabled(config=config, policy=policy):
        return a, False, "decode_gemv_disabled"
    if a.dim() != 2 or int(a.shape[0]) != 1:
        return a, False, "input_not_m1_2d"
    if q_qweight.dim() != 2 or k_qweight.dim() != 2:
        return a, False, "qk_weight_not_2d"
    if q_scales.dim() != 2 or k_scales.dim() != 2:
        return a, False, "qk_scales_not_2d"
    has_v = v_qweight is not None and v_scales is not None
    if has_v and (v_qweight.dim() != 2 or v_scales.dim() != 2):
        return a, False, "v_bad_shape"
    if int(group_size) != 32:
        return a, False, "group_size_not_32"
    k = int(a.shape[1])
    if k % 32 != 0:
        return a, False, "k_not_group_aligned"
    if k != int(q_qweight.shape[1]) * 8 or k != int(k_qweight.shape[1]) * 8:
        return a, False, "qk_k_mismatch"
    if has_v and k != int(v_qweight.shape[1]) * 8:
        return a, False, "v_k_mismatch"
    tensors = [q_qweight, k_qweight, q_scales, k_scales] + ([v_qweight, v_scales] if has_v else [])
    if any(t.device != a.device for t in tensors):
        return a, False, "device_mismatch"
    if a.dtype not in (torch.float16, torch.bfloat16):
        return a, False, f"unsupported_dtype_{str(a.dtype)}"
    try:
        c = packed_int4_symmetric_fused_qkv_m1(
            a.contiguous(), q_qweight.contiguous(), k_qweight.contiguous(),
            v_qweight.contiguous() if has_v else None, q_scales.contiguous(), k_scales.contiguous(),
            v_scales.contiguous() if has_v else None, int(group_size), config=config, policy=policy)
        expected_n = int(q_qweight.shape[0]) + int(k_qweight.shape[0]) + (int(v_qweight.shape[0]) if has_v else 0)
        if c.shape != (1, expected_n):
            return c, False, "bad_output_shape"
        return c, True, "ok"
    except Exception:
        return a, False, "kernel_exception"


def packed_int4_symmetric_fused_qkv_m2_safe(a, q_qweight, k_qweight, v_qweight, q_scales, k_scales, v_scales,
                                            group_size, *, config: Any | None = None,
                                            policy: dict | None = None) -> tuple[torch.Tensor, bool, str]:
    """Never raises; the reference's checks, order and reasons (``awq_fused_gemm.py:3592-3644``)."""
    if not awq_decode_gemv_enabled(config=config, policy=policy):
        return a, False, "decode_gemv_disabled"
    if a.dim() != 2 or int(a.shape[0]) != 2:
        return a, False, "input_not_m2_2d"
    if int(group_size) != 32 or int(a.shape[1]) % 32 != 0:
        return a, False, "unsupported_group_layout"
    tensors = [q_qweight, k_qweight, q_scales, k_scales]
    if v_qweight is not None or v_scales is not None:
        if v_qweight is None or v_scales is None:
            return a, False, "v_bad_shape"
        tensors.extend([v_qweight, v_scales])
    if any(t.dim() != 2 or t.device != a.device for t in tensors):
        return a, False, "tensor_layout_or_device"
    if any(int(a.shape[1]) != int(w.shape[1]) * 8 for w in tensors[:2]):
        return a, False, "qk_k_mismatch"
    if v_qweight is not None and int(a.shape[1]) != int(v_qweight.shape[1]) * 8:
        return a, False, "v_k_mismatch"
    try:
        c = packed_int4_symmetric_fused_qkv_m2(
            a.contiguous(), q_qweight.contiguous(), k_qweight.contiguous(),
            v_qweight.contiguous() if v_qweight is not None else None, q_scales.contiguous(),
            k_scales.contiguous(), v_scales.contiguous() if v_scales is not None else None, int(group_size),
            config=config, policy=policy)
        expected_n = (int(q_qweight.shape[0]) + int(k_qweight.shape[0])
                      + (int(v_qweight.shape[0]) if v_qweight is not None else 0))
        if c.shape != (2, expected_n):
            return c, False, "bad_output_shape"
        return c, True, "ok"
    except Exception:
        return a, False, "kernel_exception"
