"""Mixture-of-experts call surfaces of the reference, on the grouped AWQ MoE kernels.

* :func:`gemma4_moe_int4_prefill_grouped` (and ``_fused``) mirror
  ``vllm/kernels/triton/gemma4_moe_int4.py:2330-2584``: same arguments, same
  ``(out, used, reason)`` return, the validation reasons of ``_validate_batched_prefill_inputs``
  (``gemma4_moe_int4.py:1640-1708``).  Added: optional zero tensors (zero-point AWQ experts),
  group sizes 32 / 64 / 128 (the reference kernels take symmetric g = 32 only) and the
  AutoAWQ expert layout.
* :func:`fused_moe` mirrors ``vllm/model_executor/layers/fused_moe/fused_moe.py:4-77``: int4 AWQ
  experts (:class:`AWQExperts`) run the grouped kernels (routing, the gated expert MLP, the
  weighted sum); the ungated form and dense expert tensors take the reference's own expert loop.
* :func:`moe_route` is the routing alone: ``flow="logits"`` is ``fused_moe.py:12-15``'s dtype flow,
  ``flow="fp32"`` the Gemma4 router's (``gemma4/moe.py:106-123``, weights cast to the hidden
  dtype with ``weights_dtype``).

Every byte of the int4 arithmetic runs in ``libawq_w4a16.so``; there is no CPU fallback.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops
from ._lib import AWQKernelError

moe_route = ops.moe_route


@dataclass(frozen=True)
class AWQExperts:
    """An int4 expert stack.  ``layout="ref"``: qweight ``[E, N, K/8]`` (sequential nibbles),
    scales ``[E, N, K/G]``, qzeros ``[E, N, K/G/8]``; ``layout="autoawq"``: qweight
    ``[E, K, N/8]``, scales ``[E, K/G, N]``, qzeros ``[E, K/G, N/8]``.  ``qzeros=None``:
    symmetric (z = 8)."""

    qweight: torch.Tensor
    scales: torch.Tensor
    qzeros: torch.Tensor | None = None
    group_size: int | None = None
    layout: str = "ref"

    def dims(self) -> tuple[int, int, int]:
        """(E, K, N) of the unpacked stack."""
        e = int(self.qweight.shape[0])
        if self.layout == "ref":
            return e, int(self.qweight.shape[2]) * 8, int(self.qweight.shape[1])
        return e, int(self.qweight.shape[1]), int(self.qweight.shape[2]) * 8

    def group(self) -> int:
        if self.group_size:
            return int(self.group_size)
        _, k, _ = self.dims()
        ng = int(self.scales.shape[2] if self.layout == "ref" else self.scales.shape[1])
        return k // ng if ng > 0 else 0


def _ref_builder(qweight, scales, qzeros, n_rows, group_size):
    qz = qzeros[:, :n_rows] if qzeros is not None else None
    return ops.repack_experts_ref_to_autoawq(qweight[:, :n_rows], scales[:, :n_rows], qz, group_size)


_REF_CACHE = ops._DerivedCache("moe_ref_autoawq", _ref_builder)


def _as_autoawq(ex: AWQExperts, n_rows: int):
    """AutoAWQ stacks (qweight, scales, qzeros) of the first ``n_rows`` output rows."""
    g = ex.group()
    if ex.layout == "autoawq":
        n = int(ex.qweight.shape[2]) * 8
        if n == n_rows:
            return ex.qweight, ex.scales, ex.qzeros
        qz = ex.qzeros[:, :, : n_rows // 8] if ex.qzeros is not None else None
        return ex.qweight[:, :, : n_rows // 8], ex.scales[:, :, :n_rows], qz
    if ex.layout != "ref":
        raise ValueError(f"unknown expert layout {ex.layout!r}")
    return _REF_CACHE.get(ex.qweight, ex.scales, ex.qzeros, args=(int(n_rows), g))


def _expert_rows(ex: AWQExperts) -> int:
    return ex.dims()[2]


def _validate(x, topk_weights, topk_ids, gu: AWQExperts, dn: AWQExperts, intermediate: int,
              activation: str) -> tuple[bool, str]:
    """Reasons of the reference's _validate_batched_prefill_inputs (gemma4_moe_int4.py:1640-1708);
    group sizes 32 / 64 / 128 with or without zeros instead of symmetric g = 32 only."""
    if x.dim() != 2:
        return False, "input_not_2d"
    if int(x.shape[0]) <= 0:
        return False, "empty_batch"
    if topk_weights.dim() != 2 or topk_ids.dim() != 2:
        return False, "routing_not_2d"
    if tuple(topk_weights.shape) != tuple(topk_ids.shape):
        return False, "routing_shape_mismatch"
    if int(topk_weights.shape[0]) != int(x.shape[0]):
        return False, "routing_batch_mismatch"
    if str(activation).strip().lower() not in ops.MOE_ACTIVATIONS:
        return False, "unsupported_activation"
    if x.dtype not in (torch.float16, torch.bfloat16):
        return False, f"unsupported_dtype_{str(x.dtype)}"
    if gu.qweight.dim() != 3 or gu.scales.dim() != 3 or dn.qweight.dim() != 3 or dn.scales.dim() != 3:
        return False, "weights_not_expert_major"
    tensors = [topk_weights, topk_ids, gu.qweight, gu.scales, dn.qweight, dn.scales]
    tensors += [t for t in (gu.qzeros, dn.qzeros) if t is not None]
    if any(t.device != x.device for t in tensors):
        return False, "device_mismatch"
    if (gu.qzeros is None) != (dn.qzeros is None):
        return False, "zeros_mismatch"
    hidden = int(x.shape[1])
    inter = int(intermediate)
    if hidden % 32 != 0 or inter % 32 != 0:
        return False, "dims_not_group_aligned"
    e_gu, k_gu, n_gu = gu.dims()
    e_dn, k_dn, n_dn = dn.dims()
    if n_gu < 2 * inter:
        return False, "gate_up_rows_mismatch"
    if k_gu != hidden:
        return False, "gate_up_k_mismatch"
    if n_dn < hidden:
        return False, "down_rows_mismatch"
    if k_dn != inter:
        return False, "down_k_mismatch"
    if e_gu != e_dn:
        return False, "expert_count_mismatch"
    if gu.group() not in (32, 64, 128) or hidden % gu.group() != 0:
        return False, "gate_up_group_unsupported"
    if dn.group() != gu.group() or inter % dn.group() != 0:
        return False, "down_group_unsupported"
    if topk_ids.dtype not in (torch.int32, torch.int64):
        return False, "routing_ids_not_integer"
    if topk_weights.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return False, f"unsupported_routing_dtype_{str(topk_weights.dtype)}"
    return True, "ok"


def awq_moe(x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor, gate_up: AWQExperts,
            down: AWQExperts, *, intermediate_dim: int, activation: str = "silu",
            out: torch.Tensor | None = None) -> torch.Tensor:
    """Grouped MoE over int4 experts; raises on invalid input or a kernel error."""
    ok, reason = _validate(x, topk_weights, topk_ids, gate_up, down, intermediate_dim, activation)
    if not ok:
        raise ValueError(reason)
    inter, hidden = int(intermediate_dim), int(x.shape[1])
    gq, gs, gz = _as_autoawq(gate_up, 2 * inter)
    dq, ds, dz = _as_autoawq(down, hidden)
    return ops.moe(x, topk_weights, topk_ids, gq, gs, gz, dq, ds, dz, gate_up.group(), activation, out=out)


def gemma4_moe_int4_prefill_grouped(x, topk_weights, topk_ids, gate_up_qweight, gate_up_scales,
                                    down_qweight, down_scales, *, intermediate_dim: int,
                                    activation: str = "silu", block_i_override: int | None = None,
                                    gate_up_qzeros=None, down_qzeros=None, layout: str = "ref"):
    """``(out, used, reason)`` like the reference wrapper; never raises on bad input."""
    if block_i_override is not None:
        b = int(block_i_override)
        if b <= 0 or (b & (b - 1)) != 0 or b % 32 != 0:
            return x, False, "invalid_prefill_grouped_tile"
    gu = AWQExperts(gate_up_qweight, gate_up_scales, gate_up_qzeros, layout=layout)
    dn = AWQExperts(down_qweight, down_scales, down_qzeros, layout=layout)
    ok, reason = _validate(x, topk_weights, topk_ids, gu, dn, intermediate_dim, activation)
    if not ok:
        return x, False, reason
    if int(topk_ids.shape[1]) <= 0:
        return torch.zeros_like(x), True, "ok"
    try:
        out = awq_moe(x, topk_weights, topk_ids, gu, dn, intermediate_dim=intermediate_dim,
                      activation=activation)
    except (AWQKernelError, ValueError, TypeError, OSError):
        return x, False, "kernel_exception"
    return out, True, "ok"


def gemma4_moe_int4_prefill_grouped_fused(x, topk_weights, topk_ids, gate_up_qweight, gate_up_scales,
                                          down_qweight, down_scales, *, intermediate_dim: int,
                                          activation: str = "silu", block_i_override: int | None = None,
                                          block_h_override: int | None = None, gate_up_qzeros=None,
                                          down_qzeros=None, layout: str = "ref"):
    """The single-kernel variant's surface (``gemma4_moe_int4.py:2475-2584``); same kernels."""
    if block_h_override is not None:
        b = int(block_h_override)
        if b <= 0 or (b & (b - 1)) != 0:
            return x, False, "invalid_prefill_grouped_fused_tile"
    if block_i_override is not None:
        b = int(block_i_override)
        if b <= 0 or (b & (b - 1)) != 0 or b % 32 != 0:
            return x, False, "invalid_prefill_grouped_fused_tile"
    return gemma4_moe_int4_prefill_grouped(x, topk_weights, topk_ids, gate_up_qweight, gate_up_scales,
                                           down_qweight, down_scales, intermediate_dim=intermediate_dim,
                                           activation=activation, gate_up_qzeros=gate_up_qzeros,
                                           down_qzeros=down_qzeros, layout=layout)


def _dense_stack(ex: AWQExperts, n_rows: int, dtype: torch.dtype) -> torch.Tensor:
    """``[E, n_rows, K]`` dense experts in ``dtype``, dequantized by the HIP kernel (one rounding
    of ``(q - z) * s`` to fp16, bit-exact against the reference's dequant), held on the stack."""
    return _DENSE_CACHE.get(ex.qweight, ex.scales, ex.qzeros, args=(int(n_rows), ex.group(), ex.layout, dtype))


def _dense_build(qweight, scales, qzeros, n, g, layout, dt):
    outs = []
    for e in range(int(qweight.shape[0])):
        w = ops.dequant(qweight[e], scales[e], qzeros[e] if qzeros is not None else None, g, layout=layout)
        outs.append((w if layout == "ref" else w.t())[:n])
    return torch.stack(outs).to(dt).contiguous()


_DENSE_CACHE = ops._DerivedCache("moe_dense_experts", _dense_build)


def _expert_mlp(tokens: torch.Tensor, w1e: torch.Tensor, w2e: torch.Tensor, inter: int) -> torch.Tensor:
    """One expert on dense weights, the reference's dtype flow (``fused_moe.py:48-54``): the
    gated form when w1 holds gate and up (``2 * inter`` rows), otherwise SiLU alone."""
    res = torch.nn.functional.linear(tokens, w1e)
    if res.shape[-1] == 2 * inter:
        res = torch.nn.functional.silu(res[:, :inter]) * res[:, inter:]
    else:
        res = torch.nn.functional.silu(res)
    return torch.nn.functional.linear(res, w2e)


def _fused_moe_dense(hidden_states, w1, w2, topk_weights, topk_ids):
    """The reference's expert loop over dense expert tensors (``fused_moe.py:17-75``), both of its
    branches with their summation orders: routes grouped by expert and ``index_add_`` into the
    output (E < 256, K <= 4096, M <= 128), else token by token in slot order.  These are dense
    fp16 / bf16 GEMMs (hipBLASLt through ``F.linear``), outside the int4 W4A16 kernels: the form
    for callers that hand over materialised experts, kept call-compatible."""
    M, K = hidden_states.shape
    E, topk = int(w1.shape[0]), int(topk_ids.shape[1])
    inter = int(w2.shape[-1])
    out = torch.zeros_like(hidden_states)
    if not (E >= 256 or K > 4096 or M > 128):
        flat_ids = topk_ids.reshape(-1).long()
        flat_w = topk_weights.reshape(-1)
        tok = torch.arange(M, device=hidden_states.device).repeat_interleave(topk)
        sorted_ids, order = torch.sort(flat_ids)
        tok, flat_w = tok[order], flat_w[order]
        uniq, counts = torch.unique_consecutive(sorted_ids, return_counts=True)
        off = 0
        for e, c in zip(uniq.tolist(), counts.tolist()):
            idx = tok[off:off + c]
            res = _expert_mlp(hidden_states.index_select(0, idx), w1[e], w2[e], inter)
            out.index_add_(0, idx, res * flat_w[off:off + c].unsqueeze(-1))
            off += c
        return out
    for m in range(M):
        h = hidden_states[m:m + 1]
        acc = torch.zeros_like(h)
        for k in range(topk):
            e = int(topk_ids[m, k].item())
            acc += _expert_mlp(h, w1[e], w2[e], inter) * topk_weights[m, k].item()
        out[m] = acc
    return out


def fused_moe(hidden_states: torch.Tensor, w1, w2, gating_output: torch.Tensor, topk: int,
              renormalize: bool = True) -> torch.Tensor:
    """``fused_moe`` (``fused_moe.py:4-77``).

    Routing follows the reference's dtype flow (``fused_moe.py:12-15``): the softmax rounded to
    the logits dtype, top-k on those values, renormalisation in that dtype, weights in that
    dtype (:func:`moe_route` with ``flow="logits"``, a HIP kernel).
      * ``w1``, ``w2`` int4 AWQ expert stacks (:class:`AWQExperts`), ``w1`` the gate_up stack
        ``[E, 2I, H]`` (unpacked orientation), ``w2`` the down stack ``[E, H, I]``: the grouped
        W4A16 kernels (gate, up, SiLU, down and the weighted sum, fp32 sums).
      * ``w1`` an AWQ stack of ``I`` rows (the ungated form, ``fused_moe.py:52-53``): the experts
        are dequantized once by the HIP kernel (held on the stack) and run in the dense form.
      * dense ``w1 [E, 2I or I, H]`` / ``w2 [E, H, I]`` tensors (the materialised experts the
        reference's zero-point Gemma4 path passes, ``gemma4/moe.py:722-750, 788``): the
        reference's own expert loop on the device (dense GEMMs, not the int4 kernels)."""
    awq1, awq2 = isinstance(w1, AWQExperts), isinstance(w2, AWQExperts)
    if awq1 != awq2:
        raise TypeError("w1 and w2 must both be AWQExperts or both be dense expert tensors")
    H = int(hidden_states.shape[1])
    tw, tid = moe_route(gating_output, topk, renormalize, flow="logits")
    if awq1:
        _, _, n1 = w1.dims()
        _, inter, n2 = w2.dims()
        if n2 != H:
            raise ValueError("w2 rows must equal the hidden size")
        if n1 == 2 * inter:
            return awq_moe(hidden_states, tw, tid, w1, w2, intermediate_dim=inter, activation="silu")
        if n1 != inter:
            raise ValueError("w1 must hold 2 * intermediate (gated) or intermediate (ungated) rows")
        w1 = _dense_stack(w1, n1, hidden_states.dtype)
        w2 = _dense_stack(w2, n2, hidden_states.dtype)
    if w1.dim() != 3 or w2.dim() != 3 or int(w1.shape[2]) != H or int(w2.shape[1]) != H:
        raise ValueError("dense experts must be w1 [E, 2I or I, H] and w2 [E, H, I]")
    if int(w1.shape[1]) not in (int(w2.shape[2]), 2 * int(w2.shape[2])):
        raise ValueError("w1 rows must be I or 2 * I for w2 [E, H, I]")
    return _fused_moe_dense(hidden_states, w1, w2, tw.to(hidden_states.dtype), tid)
