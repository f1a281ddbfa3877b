"""One GEMM for two structurally identical AWQ projections (QKV parts, gate + up), the role
of ``try_fused_awq_pair_matmul`` (``vllm/model_executor/models/_fused_awq_pair.py:61-166``).

The two packed weights are concatenated along N once and cached on ``owner``; every call then
runs a single W4A16 GEMM whose output is ``[..., 2 * output_size]``, ``lin_a``'s columns first.
Returns ``None`` whenever the reference would (mismatched shapes, group sizes or bias presence,
high-fidelity layers, active LoRA), so callers fall back to two projections.

Layer objects need ``input_size``, ``output_size``, ``qweight``, ``scales``, ``qzeros``
(or None), ``group_size``, optionally ``bias``, ``prefix``, ``force_high_fidelity_awq`` and
``layout`` (``"ref"``: ``[N, K/8]`` tensors, concatenated along dim 0; ``"autoawq"``:
``[K, N/8]`` tensors, concatenated along dim 1).
"""
from __future__ import annotations

from typing import Any

import torch
import torch.nn as nn

from .tensor import AWQWeight, PackedInt4Weight


def _lora_is_active(lora_mapping: Any) -> bool:
    """True only when some request carries an adapter (``_fused_awq_pair.py:45-58``): a list of
    Nones (plain requests) keeps fusion on."""
    if lora_mapping is None:
        return False
    count = getattr(lora_mapping, "adapter_count", None)
    if count is not None:
        return int(count) > 0
    if isinstance(lora_mapping, (list, tuple)):
        return any(v is not None for v in lora_mapping)
    return bool(lora_mapping)


def _present(t) -> bool:
    return t is not None and t.numel() > 1


def try_fused_awq_pair_matmul(x: torch.Tensor, lin_a, lin_b, owner: nn.Module, cache_key: str, *,
                              lora_mapping: Any = None, inf_config: Any = None) -> torch.Tensor | None:
    """``cat([lin_a(x), lin_b(x)], -1)`` as one quantized GEMM, or ``None`` if not fusable."""
    if _lora_is_active(lora_mapping):
        return None
    if lin_a.input_size != lin_b.input_size or lin_a.output_size != lin_b.output_size:
        return None
    ba, bb = getattr(lin_a, "bias", None), getattr(lin_b, "bias", None)
    if (ba is None) != (bb is None):
        return None
    fused_bias = torch.cat([ba.reshape(-1), bb.reshape(-1)]).contiguous() if ba is not None else None
    if getattr(lin_a, "force_high_fidelity_awq", False) or getattr(lin_b, "force_high_fidelity_awq", False):
        return None
    qa, qb = getattr(lin_a, "qweight", None), getattr(lin_b, "qweight", None)
    if not _present(qa) or not _present(qb) or tuple(qa.shape) != tuple(qb.shape):
        return None
    if tuple(lin_a.scales.shape) != tuple(lin_b.scales.shape):
        return None
    gs = int(getattr(lin_a, "group_size", 128))
    if int(getattr(lin_b, "group_size", 128)) != gs:
        return None
    layout = getattr(lin_a, "layout", "ref")
    if getattr(lin_b, "layout", "ref") != layout:
        return None
    za, zb = getattr(lin_a, "qzeros", None), getattr(lin_b, "qzeros", None)
    zero_point = _present(za) and _present(zb) and tuple(za.shape) == tuple(zb.shape)
    symmetric = not _present(za) and not _present(zb)
    if not zero_point and not symmetric:
        return None

    cache_attr = f"_fused_awq_pair_{cache_key}"
    fused = getattr(owner, cache_attr, None)
    if fused is None:
        dim = 0 if layout == "ref" else 1
        q_cat = torch.cat([qa, qb], dim=dim).contiguous()
        s_cat = torch.cat([lin_a.scales, lin_b.scales], dim=dim).contiguous()
        prefix = getattr(lin_a, "prefix", "") or f"fused_pair:{cache_key}"
        hint = str(getattr(lin_a, "awq_profile_hint", "") or "")  # the pair's execution policy
        if zero_point:
            z_cat = torch.cat([za, zb], dim=dim).contiguous()
            fused = AWQWeight(q_cat, s_cat, z_cat, group_size=gs, prefix=prefix, profile_hint=hint, layout=layout)
        else:
            shape = getattr(lin_a, "weight_shape", None)
            shape = (2 * int(shape[0]), int(shape[1])) if shape is not None else None
            fused = PackedInt4Weight(q_cat, s_cat, group_size=gs, original_shape=shape, prefix=prefix,
                                     profile_hint=hint, layout=layout)
        setattr(owner, cache_attr, fused)

    lead = x.shape[:-1]
    out = fused.matmul(x.reshape(-1, x.shape[-1]), fused_bias, config=inf_config)
    return out.reshape(*lead, 2 * int(lin_a.output_size))


def try_fused_awq_gate_up_activation(x: torch.Tensor, gate_proj, up_proj, *, activation: str,
                                     lora_mapping: Any = None, inf_config: Any = None):
    """``act(gate_proj(x)) * up_proj(x)`` in one launch for decode (one token), or ``None``
    where the reference declines (``_fused_awq_pair.py:169-240``): active LoRA, mismatched
    sizes or group sizes, bias, high-fidelity layers, zero points, more than one token, or
    the policy switch ``awq_fused_gate_up`` off."""
    from .awq_fused_gemm import packed_int4_symmetric_fused_gate_up_m1_safe

    if _lora_is_active(lora_mapping):
        return None
    if gate_proj.input_size != up_proj.input_size or gate_proj.output_size != up_proj.output_size:
        return None
    if getattr(gate_proj, "bias", None) is not None or getattr(up_proj, "bias", None) is not None:
        return None
    if getattr(gate_proj, "force_high_fidelity_awq", False) or getattr(up_proj, "force_high_fidelity_awq", False):
        return None
    if _present(getattr(gate_proj, "qzeros", None)) or _present(getattr(up_proj, "qzeros", None)):
        return None
    qwg, qwu = getattr(gate_proj, "qweight", None), getattr(up_proj, "qweight", None)
    if not _present(qwg) or not _present(qwu) or tuple(qwg.shape) != tuple(qwu.shape):
        return None
    if tuple(gate_proj.scales.shape) != tuple(up_proj.scales.shape):
        return None
    gs = int(getattr(gate_proj, "group_size", 128))
    if int(getattr(up_proj, "group_size", 128)) != gs:
        return None
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    if int(x2.shape[0]) != 1:
        return None
    try:
        out, used, _ = packed_int4_symmetric_fused_gate_up_m1_safe(
            x2.contiguous(), qwg, qwu, gate_proj.scales, up_proj.scales, gs, activation=activation,
            config=inf_config)
        if not used:
            return None
        return out.reshape(*lead, int(gate_proj.output_size))
    except Exception:
        return None
