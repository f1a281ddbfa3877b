"""Drop-in for ``vllm/model_executor/layers/quantization/awq.py``: ``AWQConfig`` builds and
caches an ``AWQWeight`` (zero points present) or ``PackedInt4Weight`` (none) on the
layer at the first ``apply`` and forwards ``weight.matmul(x, layer.bias, config=...)``
(``awq.py:40-104``)."""
from __future__ import annotations

from typing import Any

import torch
import torch.nn as nn

from .tensor import AWQWeight, PackedInt4Weight


class QuantizationConfig:
    """Protocol of ``base_config.py:7-22``."""

    def get_name(self) -> str:
        raise NotImplementedError

    def init_layer(self, layer: nn.Module):
        raise NotImplementedError

    def apply(self, layer: nn.Module, x, *args, **kwargs):
        raise NotImplementedError

    def load_weights(self, layer: nn.Module, weights_iter):
        raise NotImplementedError


class AWQConfig(QuantizationConfig):
    def __init__(self, weight_bits: int = 4, group_size: int = 128, layout: str = "ref"):
        self.weight_bits = weight_bits
        self.group_size = group_size
        self.pack_factor = 32 // weight_bits
        self.layout = layout

    def get_name(self) -> str:
        return "awq"

    def init_layer(self, layer: nn.Module):
        layer.qweight = nn.Parameter(torch.zeros((1, 1), dtype=torch.int32), requires_grad=False)
        layer.scales = nn.Parameter(torch.zeros((1, 1), dtype=torch.float16), requires_grad=False)
        layer.qzeros = None
        layer.weight_shape = None
        if not hasattr(layer, "group_size"):
            layer.group_size = self.group_size
        layer._quant_weight = None

    def apply(self, layer: nn.Module, x: torch.Tensor, *args, **kwargs) -> torch.Tensor:
        del args
        weight = getattr(layer, "_quant_weight", None)
        if weight is None:
            qweight = getattr(layer, "qweight", None)
            prefix = getattr(layer, "prefix", "<unknown>")
            if qweight is None or qweight.numel() <= 1:
                w = getattr(layer, "weight", None)
                if w is not None and w.numel() > 1:
                    return torch.nn.functional.linear(x, w, getattr(layer, "bias", None))
                raise RuntimeError(f"AWQ weight not ready for layer '{prefix}'")
            g = int(getattr(layer, "group_size", self.group_size))
            k = qweight.shape[1] * 8 if self.layout == "ref" else qweight.shape[0]
            if k % g != 0:
                raise RuntimeError(
                    f"AWQ layout check failed for layer '{prefix}': AWQ group_size={g} does not "
                    f"divide dequantized columns ({k}) for layer '{prefix}'")
            qzeros = getattr(layer, "qzeros", None)
            kw = dict(prefix=getattr(layer, "prefix", ""),
                      high_fidelity=bool(getattr(layer, "force_high_fidelity_awq", False)),
                      profile_hint=str(getattr(layer, "awq_profile_hint", "")), layout=self.layout)
            if qzeros is not None and qzeros.numel() > 1:
                weight = AWQWeight(qweight, layer.scales, qzeros, g, **kw)
            else:
                weight = PackedInt4Weight(qweight, layer.scales, g,
                                          original_shape=getattr(layer, "weight_shape", None), **kw)
            layer._quant_weight = weight
        runtime_config = kwargs.get("inf_config", kwargs.get("config"))
        return weight.matmul(x, getattr(layer, "bias", None), config=runtime_config)

    def load_weights(self, layer: nn.Module, weights_iter, expert_idx=None, part=None):
        for name, t in weights_iter:
            if "qweight" in name:
                layer.qweight = nn.Parameter(t.contiguous(), requires_grad=False)
            elif "scales" in name:
                layer.scales = nn.Parameter(t.contiguous(), requires_grad=False)
            elif "qzeros" in name:
                layer.qzeros = nn.Parameter(t.contiguous(), requires_grad=False)
            elif "weight_shape" in name:
                layer.weight_shape = tuple(int(v) for v in t.view(-1).tolist())
            elif "bias" in name:
                layer.bias = nn.Parameter(t.contiguous(), requires_grad=False)

    @classmethod
    def from_config(cls, config: dict[str, Any]) -> "AWQConfig":
        bits = int(config.get("weight_bits", config.get("bits", 4)))
        g = int(config.get("group_size", 128))
        groups = config.get("config_groups")
        if isinstance(groups, dict):
            for grp in groups.values():
                w = grp.get("weights") if isinstance(grp, dict) else None
                if isinstance(w, dict):
                    if w.get("group_size") is not None:
                        g = int(w["group_size"])
                    if w.get("num_bits") is not None:
                        bits = int(w["num_bits"])
                    break
        return cls(weight_bits=bits, group_size=g)
