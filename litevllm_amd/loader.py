"""On-disk format adapter for AWQ linear layers: the loader step of
``vllm/model_executor/model_loader/__init__.py:551-797``, for the two int4 checkpoint formats.

* compressed-tensors pack-quantized: ``weight_packed [N, K/8]`` (sequential nibbles along K),
  ``weight_scale [N, K/G]``, optional ``weight_zero_point`` -- the reference runtime layout;
* AutoAWQ: ``qweight [K, N/8]`` (interleaved nibbles along N), ``scales [K/G, N]``,
  ``qzeros [K/G, N/8]``.

``awq_components`` collects one module's tensors under the reference's alias list
(``qweight`` <- ``weight_packed`` / ``qweight`` / ``weight``; ``scales`` <- ``weight_scale`` /
``scales``; ``qzeros`` <- ``qzeros`` / ``weight_zero``; ``bias``; ``weight_shape``) plus
``weight_zero_point``, which the reference's list does not know.  ``make_awq_weight`` infers
the layout and group size from the shapes, maps the zero point, and returns an ``AWQWeight``
(or ``PackedInt4Weight`` without zeros), optionally converted once to the AutoAWQ layout the
kernels read natively and with its decode copy prepared.
"""
from __future__ import annotations

import torch

from . import ops
from .tensor import AWQWeight, PackedInt4Weight

ALIASES = {
    "qweight": ("weight_packed", "qweight", "weight"),
    "scales": ("weight_scale", "scales"),
    "qzeros": ("qzeros", "weight_zero", "weight_zero_point"),
    "bias": ("bias",),
    "weight_shape": ("weight_shape",),
}


def awq_components(tensors: dict, prefix: str) -> dict:
    """The AWQ tensors of module ``prefix`` (keys ``prefix + "." + alias``), first alias wins."""
    comps = {}
    for key, names in ALIASES.items():
        for n in names:
            t = tensors.get(f"{prefix}.{n}" if prefix else n)
            if t is not None:
                comps[key] = t
                break
    return comps


def detect_layout(qweight: torch.Tensor, scales: torch.Tensor) -> tuple[str, int, int, int]:
    """``(layout, K, N, group_size)`` from the shapes: AutoAWQ when the scales' columns are the
    packed columns times 8 (``[K/G, N]`` against ``[K, N/8]``), the reference layout when the
    scales' rows match the weight's (``[N, K/G]`` against ``[N, K/8]``)."""
    if qweight.dim() != 2 or scales.dim() != 2:
        raise ValueError("qweight and scales must be 2-D")
    r, c = int(qweight.shape[0]), int(qweight.shape[1])
    sr, sc = int(scales.shape[0]), int(scales.shape[1])
    if sc == 8 * c and sr > 0 and r % sr == 0:
        return "autoawq", r, 8 * c, r // sr
    if sr == r and sc > 0 and (8 * c) % sc == 0:
        return "ref", 8 * c, r, (8 * c) // sc
    raise ValueError(f"cannot tell the layout of qweight {tuple(qweight.shape)} with scales {tuple(scales.shape)}")


def unsigned_zero_points(z: torch.Tensor) -> torch.Tensor:
    """Unpacked zero points as the unsigned nibbles 0..15 the packed weights are offset to.

    An ``int8`` tensor holds the signed int4 convention of compressed-tensors checkpoints (zero
    points in [-8, 7], the packed weights stored with +8): each value is shifted by +8, so that
    ``q_u - z_u == q - z``.  Any other integer dtype holds unsigned values, which must lie in
    [0, 15].  Out-of-range values raise ``ValueError`` (they cannot be packed into a nibble)."""
    if z.dtype.is_floating_point or z.dtype == torch.bool:
        raise ValueError(f"zero points must be an integer tensor, got {z.dtype}")
    zi = z.to(torch.int64)
    if z.dtype == torch.int8:
        lo, hi, off = -8, 7, 8
    else:
        lo, hi, off = 0, 15, 0
    if zi.numel() and (int(zi.min()) < lo or int(zi.max()) > hi):
        raise ValueError(f"unpacked zero points of dtype {z.dtype} must lie in [{lo}, {hi}], got "
                         f"[{int(zi.min())}, {int(zi.max())}]")
    return zi + off


def _pack_groups(z: torch.Tensor) -> torch.Tensor:
    """Unpacked zero points [N, K/G] -> the reference's packed [N, ceil(K/G/8)] (nibble i of
    word j is group 8j + i), after :func:`unsigned_zero_points`."""
    n, g = int(z.shape[0]), int(z.shape[1])
    z = unsigned_zero_points(z)
    pad = (-g) % 8
    if pad:
        z = torch.cat([z, z.new_zeros((n, pad))], 1)
    v = (z.view(n, -1, 8) << (4 * torch.arange(8, device=z.device, dtype=torch.int64))).sum(-1)
    return torch.where(v >= 2**31, v - 2**32, v).to(torch.int32)


def _zeros_for(qzeros: torch.Tensor | None, layout: str, K: int, N: int, G: int) -> torch.Tensor | None:
    if qzeros is None or qzeros.numel() <= 1:
        return None
    ng = K // G
    if layout == "autoawq":
        if tuple(qzeros.shape) != (ng, N // 8):
            raise ValueError(f"AutoAWQ qzeros must be [{ng}, {N // 8}], got {tuple(qzeros.shape)}")
        return qzeros.to(torch.int32)
    packed_cols = -(-ng // 8)
    if tuple(qzeros.shape) == (N, ng) and ng != packed_cols:
        return _pack_groups(qzeros)  # one (unpacked) zero point per group
    if tuple(qzeros.shape) == (N, packed_cols):
        return qzeros.to(torch.int32)
    raise ValueError(f"zero points must be [{N}, {-(-ng // 8)}] packed or [{N}, {ng}], got {tuple(qzeros.shape)}")


def make_awq_weight(comps: dict, *, prefix: str = "", device: torch.device | str | None = None,
                    to_autoawq: bool = True, prepare_decode: bool = False):
    """An ``AWQWeight`` (zeros present) or ``PackedInt4Weight`` (symmetric) from one module's
    checkpoint tensors.  ``to_autoawq`` converts a reference-layout weight once on the device
    (lossless); ``prepare_decode`` also builds the decode stream copy up front."""
    qweight, scales = comps["qweight"], comps["scales"]
    if device is not None:
        qweight, scales = qweight.to(device), scales.to(device)
    layout, K, N, G = detect_layout(qweight, scales)
    qzeros = comps.get("qzeros")
    if qzeros is not None and device is not None:
        qzeros = qzeros.to(device)
    qzeros = _zeros_for(qzeros, layout, K, N, G)
    qweight = qweight.to(torch.int32) if qweight.dtype != torch.int32 else qweight
    if layout == "ref" and to_autoawq and qweight.is_cuda and N % 8 == 0:
        qweight, scales, qzeros = ops.repack_ref_to_autoawq(qweight, scales, qzeros, G)
        layout = "autoawq"
    if prepare_decode and layout == "autoawq" and qweight.is_cuda:
        ops.prepare_decode_stream(qweight)
    if qzeros is None:
        shape = comps.get("weight_shape")
        shape = tuple(int(v) for v in shape.view(-1).tolist()) if shape is not None else None
        return PackedInt4Weight(qweight, scales, G, original_shape=shape, prefix=prefix, layout=layout)
    return AWQWeight(qweight, scales, qzeros, G, prefix=prefix, layout=layout)
