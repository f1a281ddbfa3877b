"""Seeded synthetic inputs for the benchmark configurations (test infrastructure).

Distributions follow the benchmark configuration: int4 weights and zeros uniform
in [0, 15] packed 8-per-int32 along N in AutoAWQ order, fp16 scales
``|N(0, 0.02)| + 1e-4`` of shape [K/G, N], fp16 activations N(0, 1); the prefill
configuration scales ~0.1% of the channels by 20 to mimic activation outliers.
"""
from __future__ import annotations

import numpy as np

from .awq_oracle import pack_awq


def make_awq_problem(M, K, N, group_size=128, seed=0, outliers=False, with_bias=False):
    """Return a dict of numpy arrays in the AutoAWQ layout.

    keys: x [M,K] f16, qweight [K,N/8] i32, qzeros [K/G,N/8] i32, scales [K/G,N] f16,
    bias [N] f16 or None.
    """
    rng = np.random.default_rng(seed)
    g = int(group_size)
    W = rng.integers(0, 16, size=(K, N), dtype=np.int32)
    Z = rng.integers(0, 16, size=(K // g, N), dtype=np.int32)
    S = (np.abs(rng.standard_normal((K // g, N), dtype=np.float32)) * 0.02 + 1e-4).astype(np.float16)
    x = rng.standard_normal((M, K), dtype=np.float32)
    if outliers:
        n_out = max(1, int(round(0.001 * K)))
        ch = rng.permutation(K)[:n_out]
        x[:, ch] *= 20.0
    x = x.astype(np.float16)
    bias = (rng.standard_normal(N, dtype=np.float32)).astype(np.float16) if with_bias else None
    return {
        "x": x,
        "qweight": pack_awq(W),
        "qzeros": pack_awq(Z),
        "scales": S,
        "bias": bias,
        "group_size": g,
    }


# The benchmark configurations (shapes only; the sweep lists are expanded here).
CONFIGS = {
    0: [dict(M=1, K=2048, N=5632)],
    1: [dict(M=m, K=4096, N=n) for m in (1, 4, 16) for n in (4096, 6144, 24576)],
    2: [dict(M=m, K=12288, N=4096, split_k=s) for m in (1, 8, 32) for s in (1, 4, 8)],
    3: [dict(M=m, K=4096, N=n, outliers=True) for m in (512, 2048) for n in (12288, 24576)],
}

MOE_CONFIG = dict(E=64, top_k=8, H=2048, I=1024, group_size=128, T=(16, 512))


def make_moe_problem(T, E=64, top_k=8, H=2048, I=1024, group_size=128, seed=0, zero_point=True):
    """Per-expert AutoAWQ-packed gate_up (K=H, N=2I) and down (K=I, N=H) weights,
    fp16 activations N(0,1) and fp16 router logits N(0,1).  ``zero_point=False`` gives
    symmetric experts (zeros None, z = 8)."""
    rng = np.random.default_rng(seed)
    g = int(group_size)

    def expert_stack(K, N):
        W = rng.integers(0, 16, size=(E, K, N), dtype=np.int32)
        Z = rng.integers(0, 16, size=(E, K // g, N), dtype=np.int32)
        S = (np.abs(rng.standard_normal((E, K // g, N), dtype=np.float32)) * 0.02 + 1e-4).astype(np.float16)
        return pack_awq(W), (pack_awq(Z) if zero_point else None), S

    gu_q, gu_z, gu_s = expert_stack(H, 2 * I)
    dn_q, dn_z, dn_s = expert_stack(I, H)
    x = rng.standard_normal((T, H), dtype=np.float32).astype(np.float16)
    logits = rng.standard_normal((T, E), dtype=np.float32).astype(np.float16)
    return {
        "x": x, "logits": logits, "top_k": top_k, "group_size": g,
        "gate_up": (gu_q, gu_z, gu_s), "down": (dn_q, dn_z, dn_s),
    }


def algorithmic_bytes(M, K, N, group_size=128, bias=False):
    """Algorithmic HBM bytes of one W4A16 GEMM (weights, scales, zeros, x, y[, bias])."""
    g = group_size
    b = K * N // 2 + (K // g) * N * 2 + (K // g) * (N // 8) * 4 + M * K * 2 + M * N * 2
    return b + (N * 2 if bias else 0)
