"""Fused RMSNorm + int4 GEMM: ``C = RMSNorm(x; norm_w, eps) @ dequant(W)^T``, the call surface of
``vllm/kernels/triton/rmsnorm_awq_fused.py:168-189`` (``rmsnorm_awq_fused_linear``).

Same arguments and result: ``x [M, K]`` fp16 or bf16, reference-layout ``qweight [N, K/8]``,
``scales [N, K/G]``, ``qzeros [N, ceil(K/G/8)]``, ``norm_w [K]``; returns ``[M, N]`` in ``x``'s
dtype.  The normalised rows are fp16 whatever ``x``'s dtype and the product is rounded to
fp16 before the store, as in the reference (``rmsnorm_awq_fused.py:168-177``); for bf16 ``x``
that fp16 result is converted to bf16.

On the device this is ``awq_w4a16_rmsnorm_gemm``: one block per row reduces the row once and
writes the normalised fp16 rows, then the dequant-GEMM kernels read them (the decode kernels
for M <= 32, the MFMA prefill kernel above), instead of every output tile recomputing the
row's sum of squares as the reference's kernel does.  The reference layout is converted once
to the kernels' layout and cached on the weight, like every other entry point here.
"""
from __future__ import annotations

import torch

from . import ops


def rmsnorm_awq_fused_linear(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
                             qzeros: torch.Tensor, group_size: int, norm_w: torch.Tensor,
                             eps: float = 1e-6) -> torch.Tensor:
    """``RMSNorm(x) @ dequant(qweight, scales, qzeros)^T`` on the HIP kernels (raises on bad
    shapes, dtypes or devices; the reference's kernel has no checks of its own)."""
    if x.dim() != 2:
        raise ValueError("x must be 2-D [M, K]")
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"unsupported dtype {x.dtype}")
    if qweight.dim() != 2 or scales.dim() != 2:
        raise ValueError("qweight and scales must be 2-D")
    K, G = int(x.shape[1]), int(group_size)
    if int(qweight.shape[1]) * 8 != K or K % G != 0:
        raise ValueError(f"K mismatch: x has {K}, qweight {tuple(qweight.shape)}, group_size {G}")
    return ops.rmsnorm_gemm(x, norm_w, float(eps), qweight, scales, qzeros, G, layout="ref")
