"""CPU restatement of the reference's AWQ W4A16 arithmetic (numpy).

TEST INFRASTRUCTURE ONLY. Product code never imports this module; only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
use it, as the checker.

Two packed layouts exist (reference paths are relative to the reference checkout):

* reference runtime layout ("ref"): ``qweight int32 [N, K/8]`` packed along K
  with sequential nibbles (nibble i of word (n, j) is W[n, 8j+i]),
  ``scales [N, K/G]``, ``qzeros int32 [N, K/G/8]`` packed the same way along the
  group axis -- ``vllm/model_executor/layers/quantization/tensor.py:842-858``,
  ``vllm/kernels/triton/awq_fused_gemm.py:1807-1839``.
* AutoAWQ "GEMM" layout ("awq"): ``qweight int32 [K, N/8]`` packed along N with
  the interleave ``order = [0, 2, 4, 6, 1, 3, 5, 7]`` (nibble i of word (k, j) is
  W[k, 8j+order[i]]), ``qzeros int32 [K/G, N/8]`` packed the same way,
  ``scales [K/G, N]``.  The reference never implements this interleave; the
  layout is fixed by the benchmark configuration, not by a reference file.

Parity status of each function is listed in its docstring; the checks that pin
it live in ``tests/test_oracle.py``.
"""
from __future__ import annotations

import numpy as np

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)
# inverse permutation: logical column offset c is stored in nibble AWQ_INV[c]
AWQ_INV = tuple(AWQ_ORDER.index(c) for c in range(8))


def _as_u32(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).view(np.uint32) if a.dtype == np.int32 else a.astype(np.uint32)


def unpack_ref(packed: np.ndarray) -> np.ndarray:
    """Sequential unpack along the last axis: ``[R, C/8] -> [R, C]`` (values 0..15).

    Follows ``tensor.py:844-849`` (shifts ``arange(0, 32, 4)``, ``& 0x0F``, ``view``).
    Pinned by: known-answer words from ``tests/test_awq_fused_gemm_numerics.py:22-35``
    and pack/unpack round trips.
    """
    u = _as_u32(packed)
    shifts = np.arange(0, 32, 4, dtype=np.uint32)
    q = (u[..., None] >> shifts) & np.uint32(0xF)
    return q.reshape(*u.shape[:-1], u.shape[-1] * 8).astype(np.int32)


def pack_ref(q: np.ndarray) -> np.ndarray:
    """Inverse of :func:`unpack_ref`: ``[R, C] (0..15) -> int32 [R, C/8]``."""
    q = np.asarray(q)
    if q.shape[-1] % 8:
        raise ValueError("last dim must be a multiple of 8")
    qq = q.reshape(*q.shape[:-1], q.shape[-1] // 8, 8).astype(np.uint32) & np.uint32(0xF)
    shifts = np.arange(0, 32, 4, dtype=np.uint32)
    words = np.bitwise_or.reduce(qq << shifts, axis=-1).astype(np.uint32)
    return words.view(np.int32)


def unpack_awq(packed: np.ndarray) -> np.ndarray:
    """AutoAWQ interleaved unpack along the last axis: ``[R, C/8] -> [R, C]``.

    Nibble i of word (r, j) holds column ``8j + AWQ_ORDER[i]``.
    Pinned by: the known answer ``0x76543210 -> [0, 4, 1, 5, 2, 6, 3, 7]``
    (hand-derived), round trips, and the half2 identity
    ``(w >> 4t) & 0x000F000F = (col 2t, col 2t+1)`` checked independently.
    """
    seq = unpack_ref(packed)  # seq[..., 8j+i] = nibble i
    out = np.empty_like(seq)
    for i, c in enumerate(AWQ_ORDER):
        out[..., c::8] = seq[..., i::8]
    return out


def pack_awq(q: np.ndarray) -> np.ndarray:
    """Inverse of :func:`unpack_awq`."""
    q = np.asarray(q)
    if q.shape[-1] % 8:
        raise ValueError("last dim must be a multiple of 8")
    seq = np.empty_like(q)
    for i, c in enumerate(AWQ_ORDER):
        seq[..., i::8] = q[..., c::8]
    return pack_ref(seq)


def repack_awq_to_ref(qweight_awq, qzeros_awq, scales_awq):
    """Lossless repack AutoAWQ ``([K,N/8], [K/G,N/8], [K/G,N])`` -> reference
    ``([N,K/8], [N,K/G/8], [N,K/G])``. Requires ``(K/G) % 8 == 0`` for the zero
    packing (the same condition ``tensor.py:850-857`` needs to broadcast).
    Pinned by: round trip with :func:`repack_ref_to_awq` and dequant equality.
    """
    W = unpack_awq(qweight_awq)            # [K, N]
    Z = unpack_awq(qzeros_awq)             # [K/G, N]
    if Z.shape[0] % 8:
        raise ValueError("reference zero layout needs (K/G) % 8 == 0")
    return (
        pack_ref(np.ascontiguousarray(W.T)),
        pack_ref(np.ascontiguousarray(Z.T)),
        np.ascontiguousarray(np.asarray(scales_awq).T),
    )


def repack_ref_to_awq(qweight_ref, qzeros_ref, scales_ref):
    """Inverse of :func:`repack_awq_to_ref`."""
    W = unpack_ref(qweight_ref)            # [N, K]
    Z = unpack_ref(qzeros_ref)             # [N, K/G]
    return (
        pack_awq(np.ascontiguousarray(W.T)),
        pack_awq(np.ascontiguousarray(Z.T)),
        np.ascontiguousarray(np.asarray(scales_ref).T),
    )


def _round_out(res_f32: np.ndarray, out_dtype: str) -> np.ndarray:
    if out_dtype == "float32":
        # unrounded: the fused kernel's M = 1 operand b (awq_fused_gemm.py:1966-1971); exact,
        # since |q - z| <= 15 and a fp16/bf16 scale carry at most 4 + 11 significant bits
        return res_f32.astype(np.float32)
    if out_dtype == "float16":
        return res_f32.astype(np.float16)
    if out_dtype == "bfloat16":
        return f32_to_bf16_bits(res_f32)
    raise ValueError(out_dtype)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 -> bfloat16 (round to nearest even); returns uint16 bit patterns.

    Matches ``Tensor.to(torch.bfloat16)`` for finite inputs (the only inputs here).
    """
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    r = (u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def dequant_ref(qweight, scales, qzeros, group_size, out_dtype="float16", zero_point=True):
    """Reference-layout dequant ``W[N, K] = RNE((q - z) * s)`` computed in float32.

    Restates ``dequantize_awq_pytorch`` (``tensor.py:835-860``: int shifts, float32
    ``(qs - zs) * scales``, one cast) and, for ``zero_point=False``,
    ``dequantize_symmetric_packed_int4_pytorch`` (``tensor.py:863-901``: z = 8).
    ``out_dtype="bfloat16"`` follows the fused Triton path's single rounding of the
    float32 product (``awq_fused_gemm.py:1966, 1976``) and returns bf16 bit patterns;
    ``out_dtype="float32"`` returns the product unrounded, the operand the fused path's
    M = 1 branch accumulates (``awq_fused_gemm.py:1966-1971``).
    Pinned by: exhaustive (q, z) x scale sweep against float64-exact products
    rounded once, the symmetric known-answer words, and the ``q == z -> +0.0`` case.
    """
    q = unpack_ref(qweight).astype(np.float32)              # [N, K]
    n, k = q.shape
    g = int(group_size)
    s = np.asarray(scales).astype(np.float32)               # [N, K/G]
    if zero_point:
        z = unpack_ref(qzeros)[:, : k // g].astype(np.float32)  # [N, K/G]
    else:
        z = np.full_like(s, 8.0)
    res = (q.reshape(n, k // g, g) - z[..., None]) * s[..., None]
    return _round_out(res.reshape(n, k), out_dtype)


def dequant_awq(qweight, scales, qzeros, group_size, out_dtype="float16", zero_point=True):
    """AutoAWQ-layout dequant ``W[K, N] = RNE((q - z) * s)`` in float32.

    Same arithmetic as :func:`dequant_ref`; only the unpack differs. Pinned by
    equality with ``dequant_ref(repack(...)).T`` and the interleave known answers.
    """
    q = unpack_awq(qweight).astype(np.float32)              # [K, N]
    k, n = q.shape
    g = int(group_size)
    s = np.asarray(scales).astype(np.float32)               # [K/G, N]
    if zero_point:
        z = unpack_awq(qzeros).astype(np.float32)           # [K/G, N]
    else:
        z = np.full_like(s, 8.0)
    res = (q.reshape(k // g, g, n) - z[:, None, :]) * s[:, None, :]
    return _round_out(res.reshape(k, n), out_dtype)


def linear_exact(x_f16, w_nk_f16, bias=None):
    """Exact oracle ``y = x @ W^T (+ bias)`` in float64 (products of fp16 values are
    exact; the float64 sum of K <= 2^16 such products carries no rounding that can
    reach fp16 precision), returned in float64 *unrounded*.

    Stands in for ``F.linear(x, W_fp16, bias)`` (``tensor.py:1147``) up to the
    summation order of the float32 accumulator. Pinned by exact-rational brute
    force on tiny shapes.
    """
    x = np.asarray(x_f16, dtype=np.float64)
    w = np.asarray(w_nk_f16, dtype=np.float64)
    y = x @ w.T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)[None, :]
    return y


def fp16_ulp(y: np.ndarray, floor: float = 1.0) -> np.ndarray:
    """Size of one fp16 ulp at ``max(|y|, floor)``.

    The floor keeps the measure meaningful near zero, where an output is the
    cancellation of terms of size ~|x||W|: there the float32 accumulator's own
    rounding (not fp16 output rounding) sets the error, so ulps of a tiny |y| would
    overstate it. ``floor=1.0`` (ulp 2^-10) is used for outputs whose RMS is >= 4.
    """
    a = np.maximum(np.abs(np.asarray(y, dtype=np.float64)), max(float(floor), 2.0 ** -14))
    e = np.floor(np.log2(a))
    return 2.0 ** (e - 10)


def error_report(y, y_ref, y_exact=None, ulp_floor=1.0):
    """max-abs, mean-relative (sum|d| / sum|ref|) and max error in fp16 ulps of ref
    (ulps taken at ``max(|ref|, ulp_floor)``, see :func:`fp16_ulp`)."""
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(y_ref, dtype=np.float64)
    d = np.abs(y - r)
    rep = {
        "max_abs": float(d.max()) if d.size else 0.0,
        "mean_rel": float(d.sum() / max(np.abs(r).sum(), 1e-30)) if d.size else 0.0,
        "max_ulp": float((d / fp16_ulp(r, ulp_floor)).max()) if d.size else 0.0,
    }
    if y_exact is not None:
        e = np.asarray(y_exact, dtype=np.float64)
        rep["max_ulp_vs_exact"] = float((np.abs(y - e) / fp16_ulp(e, ulp_floor)).max()) if d.size else 0.0
    return rep


def moe_act(g: np.ndarray, activation: str = "silu") -> np.ndarray:
    """Gate activation of the grouped MoE kernels in float64
    (``vllm/kernels/triton/gemma4_moe_int4.py:748-756``): silu ``g / (1 + e^-g)``, or the
    tanh-form GELU ``g / (1 + e^(-2 * 0.79788456 (g + 0.044715 g^3)))``."""
    g = np.asarray(g, dtype=np.float64)
    with np.errstate(over="ignore"):  # e^large = inf gives the limit g / inf = -0
        if str(activation).lower() in ("gelu", "gelu_pytorch_tanh"):
            inner = 0.7978845608028654 * (g + 0.044715 * g * g * g)
            return g / (1.0 + np.exp(-2.0 * inner))
        return g / (1.0 + np.exp(-g))


def gate_up_exact(x, w_gate, w_up, activation="silu"):
    """Dense gated MLP input ``act(x @ Wg^T) * (x @ Wu^T)`` in float64, returned unrounded:
    the M = 1 fused gate/up kernels of ``vllm/kernels/triton/awq_fused_gemm.py:1406-1506``
    sum ``x * (q - 8) * s`` in fp32 for both projections, apply the activation
    (:func:`moe_act`'s mapping, ``3040-3041``) and cast once.  ``w_gate`` / ``w_up`` are the
    dequantized [N, K] weights (pass float32 products for the unrounded ``(q - z) * s``).

    Pinned by: ``torch.nn.functional.silu`` / ``gelu(approximate="tanh")`` of float64
    ``F.linear`` products, the reference tests' own construction
    (``tests/test_gemma4_mlp_pair_fusion.py:260-356``), and the identity-weight case that
    reduces to the activation of ``x`` times ``x``.
    """
    x = np.asarray(x, dtype=np.float64)
    g = x @ np.asarray(w_gate, dtype=np.float64).T
    u = x @ np.asarray(w_up, dtype=np.float64).T
    return moe_act(g, activation) * u


def moe_grouped_exact(x_f16, topk_weights, topk_ids, w1, w2, activation="silu", inter_dtype="float16"):
    """Grouped MoE with the rounding points of the reference's grouped int4 path
    (``gemma4_moe_int4.py:686-760``: gate and up summed in fp32, ``act(gate) * up *
    route_weight`` stored in x.dtype; ``894-1030``: the down products of every route of a
    token summed in fp32, one cast at the end):

    * ``w1 [E, 2I, H]`` (rows 0..I-1 gate, I..2I-1 up) and ``w2 [E, H, I]`` are the
      dequantized expert weights (fp16 values);
    * gate/up and down sums are exact (float64);
    * the intermediate is rounded once to ``inter_dtype`` (via float32 for bfloat16);
    * the output is returned unrounded (float64);
    * routes whose id is outside ``[0, E)`` contribute nothing.

    Pinned by: agreement with the ``fused_moe`` restatement (``ref_cpu.fused_moe_cpu``, the
    torch path) within its fp16-flow error, expert-relabelling and slot-permutation
    invariance, and the single-expert case reducing to :func:`linear_exact` compositions.
    """
    x = np.asarray(x_f16, dtype=np.float64)
    w1 = np.asarray(w1)
    w2 = np.asarray(w2)
    E, I = w1.shape[0], w2.shape[2]
    ids = np.asarray(topk_ids).astype(np.int64)
    tw = np.asarray(topk_weights, dtype=np.float64)
    out = np.zeros((x.shape[0], w2.shape[1]), dtype=np.float64)
    for e in np.unique(ids):
        if e < 0 or e >= E:
            continue
        ts, js = np.nonzero(ids == e)
        gu = x[ts] @ w1[e].astype(np.float64).T
        h = moe_act(gu[:, :I], activation) * gu[:, I:] * tw[ts, js][:, None]
        if inter_dtype == "bfloat16":
            h = bf16_bits_to_f32(f32_to_bf16_bits(h.astype(np.float32))).astype(np.float64)
        else:
            h = h.astype(np.float16).astype(np.float64)
        np.add.at(out, ts, h @ w2[e].astype(np.float64).T)
    return out



def rmsnorm_rows(x, norm_w, eps):
    """The RMSNorm phase of the fused RMSNorm + int4 GEMM in float32, returned as fp16:
    ``var = sum(fp32(x)^2)``, ``rrms = rsqrt(var / K + eps)``,
    ``xn = fp16((fp32(x) * rrms) * fp32(norm_w))`` -- ``vllm/kernels/triton/
    rmsnorm_awq_fused.py:108-131`` (fp32 ``var`` and ``rrms``, two fp32 products, the cast to
    fp16 at ``:168`` whatever the input dtype).  ``x`` holds the fp16 or bf16 values (any float
    dtype), ``norm_w`` likewise.  ``var`` is the float32 rounding of the float64 sum of the
    (exact) squares -- the correctly rounded sum but in vanishingly rare cases; the reference
    adds 32-element ``tl.sum`` chunks in fp32, an order that is not part of the contract -- and
    ``rsqrt`` is correctly rounded.

    Pinned by: ``torch.nn.functional.rms_norm`` in float32 (to one fp16 ulp), the constant-row
    case (``xn = sign(x)`` exactly for unit weights), bit-exact invariance under power-of-two
    scaling of a row when ``eps = 0``, and a wrong-formula check (``sum`` in place of the mean
    fails).
    """
    x32 = np.asarray(x, dtype=np.float32)
    nw = np.asarray(norm_w, dtype=np.float32)
    k = x32.shape[1]
    var = np.sum(x32.astype(np.float64) ** 2, axis=1).astype(np.float32)
    v = var / np.float32(k) + np.float32(eps)
    rrms = (1.0 / np.sqrt(v.astype(np.float64))).astype(np.float32)
    t = (x32 * rrms[:, None]).astype(np.float32)
    return (t * nw[None, :]).astype(np.float32).astype(np.float16)


def rmsnorm_awq_linear(x, norm_w, eps, qweight, scales, qzeros, group_size, weights="float16"):
    """``rmsnorm_awq_fused_linear`` (``rmsnorm_awq_fused.py:43-189``) in float64, unrounded:
    :func:`rmsnorm_rows`, then the reference-layout weights ``(q - z) * s`` (rounded to fp16
    at ``:166-167`` for ``weights="float16"``; ``"float32"`` keeps the unrounded product the
    decode kernels use), then the exact dot products.  The caller rounds to fp16 (``:177``)
    and, for bf16 inputs, fp16 -> bf16 (the store into ``c``).

    Pinned by: the unit-RMS special case (rows of +-1, unit weights, ``eps = 0``: the
    normalised rows equal ``x`` and the result reduces to :func:`linear_exact` of the pinned
    :func:`dequant_ref`) and :func:`rmsnorm_rows`' own checks.
    """
    xn = rmsnorm_rows(x, norm_w, eps)
    w = dequant_ref(qweight, scales, qzeros, group_size, out_dtype=weights)
    return linear_exact(xn, w)
