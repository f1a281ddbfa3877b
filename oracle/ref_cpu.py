"""Torch-CPU restatement of the reference's CPU dequant+matmul path (test infrastructure).

TEST INFRASTRUCTURE ONLY: used by ``tests/`` as "the reference's own path" and by
``bench.py`` as the timed CPU baseline (``kind = "port"``). Product code never
imports it.

* :func:`dequantize_awq_cpu` restates ``dequantize_awq_pytorch``
  (``vllm/model_executor/layers/quantization/tensor.py:835-860``).
* :func:`awq_linear_cpu` restates ``AWQWeight._slow_matmul_dequant``'s dense
  fallback (``tensor.py:1124-1147``): dequantize once, ``F.linear`` after a cast to
  the activation dtype (``_match_weight_dtype``, ``tensor.py:745-748``).
* :func:`fused_moe_cpu` restates ``fused_moe``
  (``vllm/model_executor/layers/fused_moe/fused_moe.py:4-77``), both its sorted
  grouped branch and its serialized per-token branch, over dense expert weights.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def dequantize_awq_cpu(qweight: torch.Tensor, scales: torch.Tensor, qzeros: torch.Tensor,
                       group_size: int = 128) -> torch.Tensor:
    """Reference layout ``[N, K/8]`` -> fp16 ``[N, K]``; int64 shifts, float32 math."""
    n, kp = qweight.shape
    k = kp * 8
    sh = torch.arange(0, 32, 4, dtype=torch.int64)
    q = ((qweight.to(torch.int64)[..., None] >> sh) & 0xF).reshape(n, k).to(torch.float32)
    z = ((qzeros.to(torch.int64)[..., None] >> sh) & 0xF).reshape(qzeros.shape[0], -1).to(torch.float32)
    groups = k // group_size
    w = (q.reshape(n, groups, group_size) - z[:, :groups, None]) * scales.to(torch.float32)[..., None]
    return w.reshape(n, k).to(torch.float16)


def dequantize_symmetric_cpu(qweight: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """``dequantize_symmetric_packed_int4_pytorch`` (``tensor.py:863-901``): z = 8."""
    lead = tuple(qweight.shape[:-2])
    n, kp = qweight.shape[-2:]
    k = kp * 8
    sh = torch.arange(0, 32, 4, dtype=torch.int32)
    q = ((qweight.to(torch.int32)[..., None] >> sh) & 0xF).reshape(*lead, n, k).to(torch.float32) - 8.0
    w = q.reshape(*lead, n, k // group_size, group_size) * scales.to(torch.float32)[..., None]
    return w.reshape(*lead, n, k).to(torch.float16)


def awq_linear_cpu(x: torch.Tensor, qweight, scales, qzeros, group_size=128, bias=None,
                   dense_weight: torch.Tensor | None = None) -> torch.Tensor:
    """Dense fallback: ``F.linear(x, dequant(...).to(x.dtype), bias)``.

    Pass ``dense_weight`` to time the warm (LRU-cached) variant, which skips the
    dequantization exactly as ``tensor.py:1125-1129`` does.
    """
    w = dense_weight if dense_weight is not None else dequantize_awq_cpu(qweight, scales, qzeros, group_size)
    if w.dtype != x.dtype:
        w = w.to(x.dtype)
    return F.linear(x, w, bias)


def moe_routing_cpu(gating_output: torch.Tensor, topk: int, renormalize: bool = True):
    """Routing of ``fused_moe.py:12-15``: softmax in the logits dtype, top-k, renormalise."""
    rw = torch.softmax(gating_output, dim=-1)
    tw, tid = torch.topk(rw, topk, dim=-1)
    if renormalize:
        tw = tw / tw.sum(dim=-1, keepdim=True)
    return tw, tid


def _expert_mlp(tokens, w1e, w2e):
    h = F.linear(tokens, w1e)
    if h.shape[-1] == 2 * w2e.shape[-1]:
        d = h.shape[-1] // 2
        h = F.silu(h[:, :d]) * h[:, d:]
    else:
        h = F.silu(h)
    return F.linear(h, w2e)


def fused_moe_cpu(hidden_states, w1, w2, gating_output=None, topk=8, renormalize=True,
                  topk_weights=None, topk_ids=None, serialized=None):
    """Restatement of ``fused_moe`` over dense experts ``w1 [E, 2I, H]``, ``w2 [E, H, I]``.

    Routing may be given precomputed (``topk_weights``/``topk_ids``) so a GPU kernel
    and this oracle can be compared on identical routes. Output accumulates in the
    hidden dtype with ``index_add_`` in expert-sorted order (M <= 128, E < 256,
    H <= 4096) or per token in top-k order otherwise (``fused_moe.py:21``).
    ``serialized`` overrides that choice (a timing sample of a large batch keeps the
    large batch's per-token branch).
    """
    M, K = hidden_states.shape
    E = w1.shape[0]
    if topk_weights is None:
        topk_weights, topk_ids = moe_routing_cpu(gating_output, topk, renormalize)
    topk = topk_ids.shape[1]
    out = torch.zeros_like(hidden_states)
    if serialized is None:
        serialized = E >= 256 or K > 4096 or M > 128
    if not serialized:
        ids = topk_ids.reshape(-1)
        wts = topk_weights.reshape(-1)
        toks = torch.arange(M).repeat_interleave(topk)
        sorted_ids, order = torch.sort(ids)
        toks = toks[order]
        wts = wts[order]
        uniq, counts = torch.unique_consecutive(sorted_ids, return_counts=True)
        start = 0
        for e, c in zip(uniq.tolist(), counts.tolist()):
            sel = toks[start:start + c]
            gw = wts[start:start + c].unsqueeze(-1)
            start += c
            res = _expert_mlp(hidden_states.index_select(0, sel), w1[e], w2[e])
            out.index_add_(0, sel, res * gw)
    else:
        for m in range(M):
            acc = torch.zeros_like(hidden_states[m:m + 1])
            for j in range(topk):
                e = int(topk_ids[m, j].item())
                wgt = topk_weights[m, j].item()
                acc += _expert_mlp(hidden_states[m:m + 1], w1[e], w2[e]) * wgt
            out[m] = acc
    return out
