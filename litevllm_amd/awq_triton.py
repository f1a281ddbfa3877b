"""Drop-in for ``vllm/model_executor/layers/quantization/awq_triton.py`` (same names,
argument meaning and error behaviour), backed by the gfx950 HIP kernels instead of
Triton.  The module name is kept so a caller's import line does not change.
"""
from __future__ import annotations

import torch

from . import ops


def _k_of(qweight: torch.Tensor, layout: str) -> int:
    """K of a 2-D packed weight: ``[N, K/8]`` in the reference layout, ``[K, N/8]`` otherwise."""
    return int(qweight.shape[1] * 8) if layout == "ref" else int(qweight.shape[0])


def awq_fused_capability_check(input: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
                               qzeros: torch.Tensor | None, group_size: int, *,
                               layout: str = "ref") -> tuple[bool, str]:
    """Same checks and reason strings as ``awq_triton.py:7-35`` (``layout="ref"``, the reference
    layout; ``"autoawq"`` / ``"kn_seq"`` read K from ``qweight``'s first dimension)."""
    if input.device.type == "cpu":
        return False, "cpu_input"
    if qweight.device != input.device:
        return False, "device_mismatch"
    if input.dtype not in (torch.float16, torch.bfloat16):
        return False, f"unsupported_input_dtype_{str(input.dtype)}"
    if qweight.dim() != 2:
        return False, "qweight_not_2d"
    if scales.dim() != 2:
        return False, "scales_not_2d"
    if qzeros is None:
        return False, "qzeros_missing"
    if qzeros.dim() != 2:
        return False, "qzeros_not_2d"
    k = _k_of(qweight, layout)
    if int(input.shape[-1]) != k:
        return False, "k_dim_mismatch"
    if group_size <= 0:
        return False, "bad_group_size"
    if k % int(group_size) != 0:
        return False, "k_not_divisible_by_group"
    return True, "ok"


def packed_int4_fused_capability_check(input: torch.Tensor, qweight: torch.Tensor,
                                       scales: torch.Tensor, group_size: int, *,
                                       layout: str = "ref") -> tuple[bool, str]:
    """``awq_triton.py:38-61`` (symmetric mode, no zero tensor); ``layout`` as above."""
    if input.device.type == "cpu":
        return False, "cpu_input"
    if qweight.device != input.device or scales.device != input.device:
        return False, "device_mismatch"
    if input.dtype not in (torch.float16, torch.bfloat16):
        return False, f"unsupported_input_dtype_{str(input.dtype)}"
    if qweight.dim() != 2:
        return False, "qweight_not_2d"
    if scales.dim() != 2:
        return False, "scales_not_2d"
    k = _k_of(qweight, layout)
    if int(input.shape[-1]) != k:
        return False, "k_dim_mismatch"
    if group_size <= 0:
        return False, "bad_group_size"
    if k % int(group_size) != 0:
        return False, "k_not_divisible_by_group"
    return True, "ok"


def awq_dequantize_triton(qweight, scales, zeros, group_size=128, out_dtype=torch.float16,
                          *, layout: str | None = None):
    """Dequantize to a dense ``[rows, qweight.shape[1]*8]`` matrix (``awq_triton.py:150-194``).

    Without ``layout`` the geometry is inferred exactly as the reference does
    (``scales.shape[0] != rows`` means groups run along the rows, ``awq_triton.py:161``)
    and nibbles are read sequentially in both geometries (``awq_triton.py:103-104``).
    ``layout="autoawq"`` selects the AutoAWQ interleave explicitly.
    Failures raise ``RuntimeError("[AWQ_FALLBACK_DEQUANT] ...")`` like the reference.
    """
    if layout is None:
        layout = "kn_seq" if int(scales.shape[0]) != int(qweight.shape[0]) else "ref"
    try:
        return ops.dequant(qweight, scales, zeros, int(group_size), layout=layout, out_dtype=out_dtype)
    except Exception as exc:  # same wrapping as the reference
        raise RuntimeError(
            f"[AWQ_FALLBACK_DEQUANT] HIP dequant failed: {type(exc).__name__}: {exc}"
        ) from exc


def awq_gemm_triton(input, qweight, scales, zeros, group_size=128, split_k_iters=1,
                    out_dtype=torch.float16, *, layout: str = "ref"):
    """``input @ dequant(qweight).T`` (``awq_triton.py:197-209``) as one fused HIP GEMM.

    The reference accepts ``split_k_iters`` and ignores it; here a value > 1 fixes the
    K partition count and the default 1 leaves the choice to the library.  As in the
    reference, the weight is materialised in ``out_dtype`` and must match the input
    dtype for the product to be defined.
    """
    if out_dtype != input.dtype:
        raise RuntimeError(
            f"expected both operands to have the same dtype, got {input.dtype} and {out_dtype}")
    lead = input.shape[:-1]
    a2 = input.reshape(-1, input.shape[-1])
    split_k = int(split_k_iters) if int(split_k_iters) > 1 else 0
    y = ops.gemm(a2, qweight, scales, zeros, int(group_size), split_k=split_k, layout=layout)
    return y.reshape(*lead, y.shape[-1])
