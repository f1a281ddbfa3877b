"""Pins the CPU oracle (``oracle/``) before anything is checked against it.

Each check is chosen so that a plausible mistake in the oracle fails it: a wrong
nibble order, a transposed operand, pre-scaled zeros (double rounding), a dropped
zero point, a missing renormalisation. None of them re-types the oracle's formula.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import awq_oracle as O
from oracle import ref_cpu as R
from oracle.gen import make_awq_problem, algorithmic_bytes


# ---------------------------------------------------------------- known answers
# Words and scales from the reference's only hand-packed vector,
# tests/test_awq_fused_gemm_numerics.py:22-35 (symmetric, group_size=8).
KAT_WORDS = [[0x76543210, 0x6EDCBA98], [0x01234567, 0x09ABCDEF]]
KAT_SCALES = [[0.5, 0.25], [0.125, 0.75]]
# Hand-derived values, (q - 8) * s per nibble, nibble 0 first.
KAT_EXPECTED = [
    [[-4.0, -3.5, -3.0, -2.5, -2.0, -1.5, -1.0, -0.5],
     [0.0, 0.25, 0.5, 0.75, 1.0, 1.25, 1.5, -0.5]],
    [[-0.125, -0.25, -0.375, -0.5, -0.625, -0.75, -0.875, -1.0],
     [5.25, 4.5, 3.75, 3.0, 2.25, 1.5, 0.75, -6.0]],
]


def _words(ws):
    return np.array(ws, dtype=np.uint32).view(np.int32)


def test_unpack_ref_known_words():
    got = O.unpack_ref(_words([0x76543210, 0x6EDCBA98, 0x01234567, 0x09ABCDEF]))
    assert got.tolist() == [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 6,
                            7, 6, 5, 4, 3, 2, 1, 0, 15, 14, 13, 12, 11, 10, 9, 0]


def test_unpack_awq_known_word():
    # nibble i holds column order[i]; nibble values equal their index here
    assert O.unpack_awq(_words([0x76543210])).tolist() == [0, 4, 1, 5, 2, 6, 3, 7]
    assert O.unpack_awq(_words([0x000000F0])).tolist() == [0, 0, 15, 0, 0, 0, 0, 0]
    assert O.unpack_awq(_words([0x00010000])).tolist() == [0, 1, 0, 0, 0, 0, 0, 0]


def test_awq_interleave_yields_adjacent_half2_pairs():
    # The AWQ order exists so that (w >> 4t) & 0x000F000F holds columns (2t, 2t+1)
    # in its low/high 16-bit halves. Checked bit by bit, independently of unpack.
    rng = np.random.default_rng(1)
    w = rng.integers(0, 2**32, size=512, dtype=np.uint64).astype(np.uint32)
    cols = O.unpack_awq(w.view(np.int32)).reshape(-1, 8)
    for t in range(4):
        v = (w >> np.uint32(4 * t)) & np.uint32(0x000F000F)
        assert np.array_equal(v & 0xF, cols[:, 2 * t])
        assert np.array_equal(v >> 16, cols[:, 2 * t + 1])


def test_symmetric_dequant_known_answers():
    q = _words(KAT_WORDS).reshape(2, 2, 1)
    s = np.array(KAT_SCALES, dtype=np.float16).reshape(2, 2, 1)
    for e in range(2):
        w = O.dequant_ref(q[e], s[e], None, 8, zero_point=False)
        assert w.dtype == np.float16
        assert w.astype(np.float64).tolist() == KAT_EXPECTED[e]
        # the torch restatement of the reference CPU path agrees bit for bit
        wt = R.dequantize_symmetric_cpu(torch.from_numpy(q[e]), torch.from_numpy(s[e]), 8)
        assert np.array_equal(wt.numpy().view(np.uint16), w.view(np.uint16))


# ------------------------------------------------------------- round trips
@pytest.mark.parametrize("shape", [(3, 8), (16, 64), (5, 40)])
def test_pack_unpack_round_trip(shape):
    rng = np.random.default_rng(2)
    q = rng.integers(0, 16, size=shape, dtype=np.int32)
    assert np.array_equal(O.unpack_ref(O.pack_ref(q)), q)
    assert np.array_equal(O.unpack_awq(O.pack_awq(q)), q)
    w = rng.integers(0, 2**32, size=(shape[0], shape[1] // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
    assert np.array_equal(O.pack_ref(O.unpack_ref(w)), w)
    assert np.array_equal(O.pack_awq(O.unpack_awq(w)), w)


def test_repack_is_lossless_and_dequant_consistent():
    p = make_awq_problem(M=1, K=256, N=64, group_size=32, seed=3)
    qr, zr, sr = O.repack_awq_to_ref(p["qweight"], p["qzeros"], p["scales"])
    assert qr.shape == (64, 32) and zr.shape == (64, 1) and sr.shape == (64, 8)
    qa, za, sa = O.repack_ref_to_awq(qr, zr, sr)
    assert np.array_equal(qa, p["qweight"]) and np.array_equal(za, p["qzeros"])
    assert np.array_equal(sa, p["scales"])
    wa = O.dequant_awq(p["qweight"], p["scales"], p["qzeros"], 32)      # [K, N]
    wr = O.dequant_ref(qr, sr, zr, 32)                                   # [N, K]
    assert np.array_equal(wa.T.view(np.uint16), wr.view(np.uint16))


def test_repack_brute_force_small():
    # element-by-element restatement of the two layouts with Python ints
    rng = np.random.default_rng(4)
    K, N = 16, 16
    W = rng.integers(0, 16, size=(K, N))
    awq = O.pack_awq(W.astype(np.int32)).view(np.uint32)
    ref = O.repack_awq_to_ref(O.pack_awq(W.astype(np.int32)),
                              O.pack_awq(np.zeros((8, N), np.int32)),
                              np.ones((8, N), np.float16))[0].view(np.uint32)
    order = [0, 2, 4, 6, 1, 3, 5, 7]
    for k in range(K):
        for n in range(N):
            i = order.index(n % 8)
            assert (int(awq[k, n // 8]) >> (4 * i)) & 0xF == W[k, n]
            assert (int(ref[n, k // 8]) >> (4 * (k % 8))) & 0xF == W[k, n]


# ---------------------------------------------------------- dequant rounding
def _scale_set():
    rng = np.random.default_rng(5)
    s = (np.abs(rng.standard_normal(4000)) * 0.02 + 1e-4).astype(np.float16)
    edge = np.array([1e-4, 6.103515625e-05, 2.0**-10, 0.0999, 0.5, 1.0, 1.999, 0.33325,
                     np.float16(np.nextafter(np.float16(0.02), np.float16(1)))], dtype=np.float16)
    return np.concatenate([s, edge])


def test_dequant_single_rounding_exhaustive_q_z():
    """Every (q, z) pair against many scales: W must equal RNE of the exact
    product (q - z) * s. A pre-scaled-zero oracle (q*s - z*s, or an fma) fails."""
    scales = _scale_set()
    G = 16
    n_groups = 16          # zero word of 8 nibbles x 2
    K = G * n_groups
    q = np.tile(np.arange(16, dtype=np.int32), K // 16)            # q = k % 16
    Q = np.broadcast_to(q, (16, K)).copy()                           # 16 rows
    Z = (np.arange(16)[:, None] + np.arange(n_groups)[None, :]) % 16  # all z per row
    qw = O.pack_ref(Q)
    qz = O.pack_ref(Z.astype(np.int32))
    for start in range(0, scales.size - 256 + 1, 256):
        S = scales[start:start + 256].reshape(16, 16)
        W = O.dequant_ref(qw, S, qz, G)
        exact = (Q.reshape(16, n_groups, G) - Z[..., None]).astype(np.float64) * S.astype(np.float64)[..., None]
        want = exact.reshape(16, K).astype(np.float16)   # one rounding from the exact value
        assert np.array_equal(W.view(np.uint16), want.view(np.uint16))
    # q == z gives +0.0 (never -0.0) for positive scales
    zero_mask = Q.reshape(16, n_groups, G) == Z[..., None]
    assert not np.signbit(W.reshape(16, n_groups, G)[zero_mask]).any()


def test_dequant_float32_is_the_exact_product():
    """The unrounded operand (the fused path's M = 1 ``b``): every (q, z) pair against many
    scales equals the float64 product exactly, and one fp16 rounding of it reproduces the
    fp16 dequant bit for bit."""
    scales = _scale_set()
    G, n_groups = 16, 16
    K = G * n_groups
    Q = np.broadcast_to(np.tile(np.arange(16, dtype=np.int32), K // 16), (16, K)).copy()
    Z = (np.arange(16)[:, None] + np.arange(n_groups)[None, :]) % 16
    qw, qz = O.pack_ref(Q), O.pack_ref(Z.astype(np.int32))
    for start in range(0, scales.size - 256 + 1, 256):
        S = scales[start:start + 256].reshape(16, 16)
        W32 = O.dequant_ref(qw, S, qz, G, out_dtype="float32")
        exact = ((Q.reshape(16, n_groups, G) - Z[..., None]).astype(np.float64)
                 * S.astype(np.float64)[..., None]).reshape(16, K)
        assert W32.dtype == np.float32 and np.array_equal(W32.astype(np.float64), exact)
        W16 = O.dequant_ref(qw, S, qz, G)
        assert np.array_equal(W32.astype(np.float16).view(np.uint16), W16.view(np.uint16))
    # the AutoAWQ unpack agrees with the reference one on the unrounded values too
    p = make_awq_problem(M=1, K=256, N=64, group_size=32, seed=4)
    qr, zr, sr = O.repack_awq_to_ref(p["qweight"], p["qzeros"], p["scales"])
    assert np.array_equal(O.dequant_awq(p["qweight"], p["scales"], p["qzeros"], 32, out_dtype="float32"),
                          O.dequant_ref(qr, sr, zr, 32, out_dtype="float32").T)


def test_prescaled_zero_variant_is_caught():
    """Plants the classic mistake (q*s - z*s in fp16) and shows the exhaustive
    check above would reject it."""
    s = _scale_set()[:256].astype(np.float16)
    q = np.arange(16, dtype=np.float16)[:, None, None]
    z = np.arange(16, dtype=np.float16)[None, :, None]
    bad = (q * s - z * s).astype(np.float16)          # two roundings
    good = ((q.astype(np.float64) - z) * s.astype(np.float64)).astype(np.float16)
    assert (bad.view(np.uint16) != good.view(np.uint16)).any()


def test_bf16_dequant_single_rounding():
    scales = _scale_set()[:256].reshape(16, 16)
    G, K = 16, 256
    Q = np.broadcast_to(np.tile(np.arange(16, dtype=np.int32), K // 16), (16, K)).copy()
    Z = (np.arange(16)[:, None] + np.arange(16)[None, :]) % 16
    W = O.dequant_ref(O.pack_ref(Q), scales, O.pack_ref(Z.astype(np.int32)), G, out_dtype="bfloat16")
    exact = ((Q.reshape(16, 16, G) - Z[..., None]) * scales.astype(np.float64)[..., None]).reshape(16, K)
    want = torch.from_numpy(exact).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(W, want)


def test_cpu_port_matches_numpy_oracle_bitwise():
    p = make_awq_problem(M=3, K=1024, N=256, group_size=128, seed=6)
    qr, zr, sr = O.repack_awq_to_ref(p["qweight"], p["qzeros"], p["scales"])
    w_np = O.dequant_ref(qr, sr, zr, 128)
    w_t = R.dequantize_awq_cpu(torch.from_numpy(qr), torch.from_numpy(sr), torch.from_numpy(zr), 128)
    assert np.array_equal(w_t.numpy().view(np.uint16), w_np.view(np.uint16))


# ------------------------------------------------------------------- GEMM
def test_linear_exact_against_rationals():
    rng = np.random.default_rng(7)
    M, K, N = 2, 16, 8
    x = rng.standard_normal((M, K)).astype(np.float16)
    w = (rng.standard_normal((N, K)) * 0.1).astype(np.float16)
    b = rng.standard_normal(N).astype(np.float16)
    y = O.linear_exact(x, w, b)
    for m in range(M):
        for n in range(N):
            exact = sum(Fraction(float(x[m, k])) * Fraction(float(w[n, k])) for k in range(K)) + Fraction(float(b[n]))
            assert Fraction(y[m, n]) == exact


def test_linear_exact_orientation_is_caught():
    # W[N, K] vs a transposed operand: distinct shapes make a swap fail loudly,
    # and a square case shows the numbers differ.
    rng = np.random.default_rng(8)
    x = rng.standard_normal((4, 8)).astype(np.float16)
    w = rng.standard_normal((8, 8)).astype(np.float16)
    assert not np.allclose(O.linear_exact(x, w), O.linear_exact(x, w.T))
    with pytest.raises(ValueError):
        O.linear_exact(x, rng.standard_normal((8, 5)).astype(np.float16))


def test_reference_cpu_linear_within_one_ulp_of_exact():
    p = make_awq_problem(M=4, K=2048, N=512, group_size=128, seed=9)
    qr, zr, sr = O.repack_awq_to_ref(p["qweight"], p["qzeros"], p["scales"])
    y = R.awq_linear_cpu(torch.from_numpy(p["x"]), torch.from_numpy(qr), torch.from_numpy(sr),
                         torch.from_numpy(zr), 128).numpy()
    w = O.dequant_ref(qr, sr, zr, 128)
    ye = O.linear_exact(p["x"], w)
    rep = O.error_report(y, ye)
    assert rep["max_ulp"] <= 1.0, rep


def test_algorithmic_bytes_config0():
    # 5,767,168 + 180,224 + 45,056 + 4,096 + 11,264
    assert algorithmic_bytes(1, 2048, 5632) == 6_007_808


# -------------------------------------------------------------------- MoE
def _moe_dense_problem(T, E, H, I, topk, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).half()
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.05).half()
    w2 = (torch.randn(E, H, I, generator=g) * 0.05).half()
    logits = torch.randn(T, E, generator=g).half()
    return x, w1, w2, logits


def _moe_brute_force(x, w1, w2, tw, tid):
    """float64 per-token loop: y_t = sum_j w_tj * down_e(silu(gate_e x) * up_e x)."""
    T = x.shape[0]
    I = w2.shape[2]
    out = np.zeros((T, w2.shape[1]))
    xd, w1d, w2d = x.double().numpy(), w1.double().numpy(), w2.double().numpy()
    for t in range(T):
        for j in range(tid.shape[1]):
            e = int(tid[t, j])
            h = w1d[e] @ xd[t]
            a = h[:I] / (1.0 + np.exp(-h[:I])) * h[I:]
            out[t] += float(tw[t, j]) * (w2d[e] @ a)
    return out


@pytest.mark.parametrize("T", [6, 130])
def test_fused_moe_port_against_brute_force(T):
    E, H, I, topk = 8, 64, 32, 2
    x, w1, w2, logits = _moe_dense_problem(T, E, H, I, topk, seed=10)
    tw, tid = R.moe_routing_cpu(logits, topk)
    y = R.fused_moe_cpu(x, w1, w2, logits, topk).double().numpy()
    want = _moe_brute_force(x, w1, w2, tw, tid)
    # fp16 intermediates and fp16 accumulation: a few fp16 ulps of |y|
    floor = float(np.sqrt(np.mean(want ** 2)))   # ulps of the output RMS
    assert np.max(np.abs(y - want) / O.fp16_ulp(want, floor)) <= 8.0
    # planted mistake: dropping the renormalisation is far outside that band
    tw_bad = torch.softmax(logits.float(), -1).topk(topk, -1).values
    bad = _moe_brute_force(x, w1, w2, tw_bad, tid)
    assert np.max(np.abs(bad - want) / O.fp16_ulp(want, floor)) > 100.0


def test_fused_moe_single_expert_reduces_to_dense_mlp():
    T, E, H, I = 5, 1, 32, 16
    x, w1, w2, logits = _moe_dense_problem(T, E, H, I, 1, seed=11)
    y = R.fused_moe_cpu(x, w1, w2, logits, 1)
    h = torch.nn.functional.linear(x, w1[0])
    want = torch.nn.functional.linear(torch.nn.functional.silu(h[:, :I]) * h[:, I:], w2[0])
    assert torch.equal(y, want)


# ---------------------------------------------------------------- grouped MoE oracle
def test_moe_act_matches_library_routines():
    g = torch.linspace(-12, 12, 2001, dtype=torch.float64)
    assert np.allclose(O.moe_act(g.numpy(), "silu"), torch.nn.functional.silu(g).numpy(), rtol=1e-12, atol=1e-15)
    ref = torch.nn.functional.gelu(g, approximate="tanh").numpy()
    assert np.allclose(O.moe_act(g.numpy(), "gelu_pytorch_tanh"), ref, rtol=1e-12, atol=1e-15)


def test_moe_grouped_exact_against_fused_moe_port():
    T, E, H, I, topk = 40, 8, 64, 32, 3
    x, w1, w2, logits = _moe_dense_problem(T, E, H, I, topk, seed=21)
    tw, tid = R.moe_routing_cpu(logits, topk)
    ported = R.fused_moe_cpu(x, w1, w2, topk_weights=tw, topk_ids=tid).double().numpy()
    exact = O.moe_grouped_exact(x.numpy(), tw.float().numpy(), tid.numpy(), w1.numpy(), w2.numpy())
    floor = float(np.sqrt(np.mean(exact ** 2)))
    # the port rounds every intermediate to fp16 and accumulates in fp16: a few ulps
    assert np.max(np.abs(ported - exact) / O.fp16_ulp(exact, floor)) <= 8.0
    # planted mistake: gate and up halves swapped is far outside that band
    w1_swapped = torch.cat([w1[:, I:], w1[:, :I]], dim=1)
    bad = O.moe_grouped_exact(x.numpy(), tw.float().numpy(), tid.numpy(), w1_swapped.numpy(), w2.numpy())
    assert np.max(np.abs(bad - exact) / O.fp16_ulp(exact, floor)) > 100.0


def test_moe_grouped_exact_invariances():
    T, E, H, I, topk = 24, 6, 64, 32, 3
    x, w1, w2, logits = _moe_dense_problem(T, E, H, I, topk, seed=22)
    tw, tid = R.moe_routing_cpu(logits, topk)
    xs, tws, tids = x.numpy(), tw.float().numpy(), tid.numpy()
    base = O.moe_grouped_exact(xs, tws, tids, w1.numpy(), w2.numpy())
    # relabelling experts (ids and stacks together) changes nothing
    perm = np.random.default_rng(3).permutation(E)
    inv = np.argsort(perm)
    relab = O.moe_grouped_exact(xs, tws, perm[tids], w1.numpy()[inv], w2.numpy()[inv])
    assert np.allclose(relab, base, rtol=1e-12, atol=1e-12)
    # permuting a token's slots (id and weight together) changes nothing
    sp = np.random.default_rng(4).permuted(np.tile(np.arange(topk), (T, 1)), axis=1)
    slot = O.moe_grouped_exact(xs, np.take_along_axis(tws, sp, 1), np.take_along_axis(tids, sp, 1),
                               w1.numpy(), w2.numpy())
    assert np.allclose(slot, base, rtol=1e-12, atol=1e-12)
    # pairing ids with the wrong weights is caught
    bad = O.moe_grouped_exact(xs, tws[:, ::-1], tids, w1.numpy(), w2.numpy())
    assert not np.allclose(bad, base, rtol=1e-3)
    # out-of-range ids contribute nothing
    tids_oob = tids.copy()
    tids_oob[:, 0] = E + 5
    part = O.moe_grouped_exact(xs, tws, tids_oob, w1.numpy(), w2.numpy())
    only0 = O.moe_grouped_exact(xs, tws[:, :1], tids[:, :1], w1.numpy(), w2.numpy())
    assert np.allclose(part + only0, base, rtol=1e-9, atol=1e-9)


def test_moe_grouped_exact_single_expert_is_a_dense_mlp():
    T, E, H, I = 7, 1, 64, 32
    x, w1, w2, _ = _moe_dense_problem(T, E, H, I, 1, seed=23)
    ones, zeros = np.ones((T, 1), np.float32), np.zeros((T, 1), np.int64)
    y = O.moe_grouped_exact(x.numpy(), ones, zeros, w1.numpy(), w2.numpy())
    gu = O.linear_exact(x.numpy(), w1.numpy()[0])
    h = (torch.nn.functional.silu(torch.from_numpy(gu[:, :I])).numpy() * gu[:, I:]).astype(np.float16)
    assert np.allclose(y, O.linear_exact(h, w2.numpy()[0]), rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- RMSNorm prologue oracle
@pytest.mark.parametrize("K", [8, 128, 4096])
def test_rmsnorm_rows_matches_torch_rms_norm(K):
    g = torch.Generator().manual_seed(K)
    x = (torch.randn(6, K, generator=g) * 3).to(torch.float16)
    nw = (1 + 0.5 * torch.randn(K, generator=g)).to(torch.float16)
    want = torch.nn.functional.rms_norm(x.float(), (K,), weight=nw.float(), eps=1e-6).to(torch.float16)
    got = O.rmsnorm_rows(x.numpy(), nw.numpy(), 1e-6)
    diff = np.abs(got.astype(np.float64) - want.numpy().astype(np.float64))
    ulp = O.fp16_ulp(want.numpy().astype(np.float64), floor=2.0 ** -14)
    assert (diff / ulp).max() <= 1.0
    assert (diff == 0).mean() > 0.97
    # a plausible mistake, the sum of squares in place of the mean, is far off
    xd = x.double().numpy()
    wrong = xd / np.sqrt((xd ** 2).sum(1, keepdims=True)) * nw.double().numpy()
    assert np.abs(got.astype(np.float64) - wrong).max() > 0.1


def test_rmsnorm_rows_special_cases():
    K = 256
    row = np.full((1, K), 3.0, dtype=np.float16)
    assert np.array_equal(O.rmsnorm_rows(row, np.ones(K), 0.0), np.ones((1, K), np.float16))
    assert np.array_equal(O.rmsnorm_rows(-row, np.ones(K), 0.0), -np.ones((1, K), np.float16))
    # eps enters: a row of zeros normalises to zeros, a tiny row is damped
    assert np.array_equal(O.rmsnorm_rows(np.zeros((1, K), np.float16), np.ones(K), 1e-6), np.zeros((1, K), np.float16))
    tiny = np.full((1, K), 2.0 ** -10, dtype=np.float16)
    assert O.rmsnorm_rows(tiny, np.ones(K), 1e-2).max() < 0.05
    # power-of-two scaling of a row leaves the result unchanged, bit for bit (eps = 0)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, K)).astype(np.float16)
    nw = rng.uniform(0.5, 1.5, K).astype(np.float16)
    base = O.rmsnorm_rows(x, nw, 0.0)
    for j in (-4, 3):
        assert np.array_equal(O.rmsnorm_rows((x.astype(np.float32) * 2.0 ** j).astype(np.float16), nw, 0.0), base)


def test_rmsnorm_awq_linear_unit_rms_reduces_to_linear():
    N, K, G = 24, 256, 32
    rng = np.random.default_rng(5)
    x = np.where(rng.random((3, K)) < 0.5, -1.0, 1.0).astype(np.float16)
    qw = O.pack_ref(rng.integers(0, 16, (N, K)))
    qz = O.pack_ref(rng.integers(0, 16, (N, K // G)))
    sc = rng.uniform(0.001, 0.02, (N, K // G)).astype(np.float16)
    got = O.rmsnorm_awq_linear(x, np.ones(K, np.float16), 0.0, qw, sc, qz, G)
    want = O.linear_exact(x, O.dequant_ref(qw, sc, qz, G))
    assert np.array_equal(got, want)
    # the normalisation is not skipped: doubling x leaves the result unchanged
    assert np.array_equal(O.rmsnorm_awq_linear(2 * x, np.ones(K, np.float16), 0.0, qw, sc, qz, G), want)
