"""GPU parity of the grouped AWQ MoE path (routing, gate_up + activation, down, combine)
against the CPU oracle: ``oracle.awq_oracle.moe_grouped_exact`` (float64 sums, the
intermediate rounded once, the reference grouped kernel's rounding points, with the weights
the serving kernel multiplies -- see ``_mfma_path``) and the ``fused_moe`` restatement
(``oracle.ref_cpu.fused_moe_cpu``).

Bar: the kernel's output within 4 fp16 ulps (ulps at max(|y|, RMS(y))) of the exact oracle
and mean relative error <= 2e-4; bitwise reproducible across calls.  The intermediate is
rounded to fp16 (the reference keeps it in x.dtype), so a float32 gate/up sum that differs
from the exact one in its last bits can land an intermediate value one fp16 ulp away from the
oracle's; that ulp times its down weight moves an output by up to a few ulps (e.g. h = 9.15
vs 9.14 with weight 0.593: 2.4 ulps at the RMS scale -- reproduced bit for bit by a float32
emulation of the kernel's arithmetic on the CPU).  The mean error stays at the output
rounding's level.
"""
import numpy as np
import pytest
import torch

from litevllm_amd import moe as MOE
from litevllm_amd import ops
from oracle import awq_oracle as O
from oracle import ref_cpu as R
from oracle.gen import make_moe_problem

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _dev(a):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _problem(T, E, H, I, topk, G, zp=True, seed=0):
    p = make_moe_problem(T, E=E, top_k=topk, H=H, I=I, group_size=G, seed=seed, zero_point=zp)
    gq, gz, gs = p["gate_up"]
    dq, dz, ds = p["down"]
    return p, dict(gq=_dev(gq), gz=_dev(gz), gs=_dev(gs), dq=_dev(dq), dz=_dev(dz), ds=_dev(ds))


def _dense_experts(d, G):
    """Dequantized stacks in the oracle's orientation, w1 [E, 2I, H], w2 [E, H, I] (fp16), from
    the device dequant kernel, which is bit-exact against the oracle's dequant."""
    E = d["gq"].shape[0]
    w1 = torch.stack([ops.dequant(d["gq"][e], d["gs"][e], None if d["gz"] is None else d["gz"][e], G,
                                  layout="autoawq").t() for e in range(E)])
    w2 = torch.stack([ops.dequant(d["dq"][e], d["ds"][e], None if d["dz"] is None else d["dz"][e], G,
                                  layout="autoawq").t() for e in range(E)])
    return w1.cpu().numpy(), w2.cpu().numpy()


def _mfma_path(T, E, H, I, topk, G=128):
    """The grouped MFMA kernels serve at least 16 routes per expert when H and I are multiples
    of 64 and the group size is a power of two; they multiply weights rounded to the activation
    dtype (each dequantized operand feeds up to six 16-route MFMA tiles).  The decode-structured
    kernels serve the rest and multiply the exact integers q - z, scaling each group's fp32 sum
    once: unrounded weights, as the reference's int4 kernels (gemma4_moe_int4.py:736-742)."""
    return T * topk >= 16 * E and H % 64 == 0 and I % 64 == 0 and G & (G - 1) == 0


def _unrounded_experts(p, G):
    """w1 [E, 2I, H], w2 [E, H, I] as float32 (q - z) * s, never rounded."""
    gq, gz, gs = p["gate_up"]
    dq, dz, ds = p["down"]
    E = gq.shape[0]
    zp = gz is not None
    f = lambda q, s, z: O.dequant_awq(q, s, z, G, out_dtype="float32", zero_point=zp).T
    w1 = np.stack([f(gq[e], gs[e], gz[e] if zp else None) for e in range(E)])
    w2 = np.stack([f(dq[e], ds[e], dz[e] if zp else None) for e in range(E)])
    return w1, w2


def _experts_used(p, d, G, mfma):
    return _dense_experts(d, G) if mfma else _unrounded_experts(p, G)


def _route_cpu(logits, topk):
    p = torch.softmax(logits.float(), dim=-1)
    w, i = torch.topk(p, topk, dim=-1)
    return w / w.sum(-1, keepdim=True).clamp_min(1e-8), i


def _check(y, exact, what):
    floor = float(np.sqrt(np.mean(exact ** 2)))
    rep = O.error_report(y, exact, ulp_floor=floor)
    print(what, rep, flush=True)
    assert rep["max_ulp"] <= 4.0 and rep["mean_rel"] <= 2e-4, (what, rep)


def test_dequant_matches_oracle_for_expert_slices():
    # the full-size tests below take the dense experts from the device dequant; pin it here
    p, d = _problem(2, 3, 256, 128, 2, 64, seed=1)
    gq, gz, gs = p["gate_up"]
    for e in range(3):
        w = ops.dequant(d["gq"][e], d["gs"][e], d["gz"][e], 64, layout="autoawq").cpu().numpy()
        ref = O.dequant_awq(gq[e], gs[e], gz[e], 64)
        assert np.array_equal(w.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("T,E,topk", [(1, 8, 2), (37, 64, 8), (300, 16, 4), (20, 128, 8), (9, 256, 6)])
def test_route_matches_fp32_torch(T, E, topk):
    g = torch.Generator().manual_seed(T)
    logits = torch.randn(T, E, generator=g).half()
    w, ids = ops.moe_route(logits.to(DEV), topk)
    wr, ir = _route_cpu(logits, topk)
    assert torch.equal(ids.cpu().long(), ir)
    assert torch.allclose(w.cpu(), wr, rtol=2e-6, atol=1e-7)
    # weights of a token sum to one
    assert torch.allclose(w.sum(-1).cpu(), torch.ones(T), atol=1e-6)


def test_route_ties_pick_lower_expert():
    logits = torch.zeros(3, 16, dtype=torch.float16)
    w, ids = ops.moe_route(logits.to(DEV), 4)
    assert ids.cpu().tolist() == [[0, 1, 2, 3]] * 3
    assert torch.allclose(w.cpu(), torch.full((3, 4), 0.25))


def test_route_partial_ties_straddle_the_cut():
    """Equal probabilities on both sides of the k-th place: the lower expert ids are taken, in
    id order among equals (E <= 64 ranks lanes in one pass, larger E repeats the arg-max)."""
    for E in (32, 64, 96):
        logits = torch.zeros(4, E, dtype=torch.float16)
        logits[:, [5, 9, 17, 30]] = 2.0
        logits[:, [3, 12, 20, 25]] = 1.0  # three of these four make the top 7
        w, ids = ops.moe_route(logits.to(DEV), 7)
        sel = [5, 9, 17, 30, 3, 12, 20]
        assert ids.cpu().tolist() == [sel] * 4, E
        p = torch.softmax(logits.float(), dim=-1)[:, sel]  # torch.topk leaves tie order open
        assert torch.allclose(w.cpu(), p / p.sum(-1, keepdim=True), rtol=2e-6, atol=1e-7)


CASES = [
    # T, E, H, I, topk, G, zero point, activation
    (1, 4, 128, 64, 2, 32, True, "silu"),
    (6, 8, 256, 128, 2, 64, False, "silu"),
    (16, 64, 512, 256, 8, 128, True, "silu"),
    (100, 8, 256, 128, 2, 128, True, "gelu_pytorch_tanh"),   # ~25 routes per expert
    (200, 4, 256, 160, 2, 32, True, "silu"),                # ~100 routes per expert, I % 64 != 0
    # >= 16 routes per expert with H, I % 64 == 0: the grouped MFMA kernels
    (64, 4, 256, 128, 2, 32, False, "silu"),                # 32 routes/expert, 2 groups per k-stage
    (128, 8, 512, 192, 4, 64, True, "gelu_pytorch_tanh"),   # partial gate tile (I = 192)
    (300, 16, 256, 256, 4, 128, True, "silu"),              # ~75 routes/expert: 2 row tiles
    # Gemma4's symmetric group-32 experts (z = 8, tanh GELU) at a decode batch
    (16, 64, 512, 256, 8, 32, False, "gelu_pytorch_tanh"),
    # 128 experts, 8 and 12.5 routes each: the stream kernels with one and two route tiles
    (128, 128, 256, 128, 8, 64, True, "silu"),
    (200, 128, 256, 128, 8, 128, True, "silu"),
    # 128 experts at 32 routes each: the grouped tile kernels, whose tile search passes over
    # the experts 64 at a time
    (512, 128, 256, 128, 8, 128, True, "silu"),
    # 4800 routes: the route lists kernel's rounds past the 4096 ids it requests at once
    (600, 64, 256, 128, 8, 128, True, "silu"),
    # 96 routes per expert (six token tiles: the body that forms each nibble pair's zeros from
    # the held zero word), symmetric and with groups of 32 rows (a new group every k-step)
    (192, 4, 256, 128, 2, 128, False, "silu"),
    (192, 4, 256, 128, 2, 32, True, "gelu_pytorch_tanh"),
]


@pytest.mark.parametrize("T,E,H,I,topk,G,zp,act", CASES)
def test_moe_vs_exact_oracle(T, E, H, I, topk, G, zp, act):
    p, d = _problem(T, E, H, I, topk, G, zp, seed=T + E)
    logits = torch.from_numpy(p["logits"])
    tw, tid = _route_cpu(logits, topk)
    x = _dev(p["x"])
    y = ops.moe(x, tw.to(DEV), tid.to(DEV), d["gq"], d["gs"], d["gz"], d["dq"], d["ds"], d["dz"], G, act)
    y2 = ops.moe(x, tw.to(DEV), tid.to(DEV), d["gq"], d["gs"], d["gz"], d["dq"], d["ds"], d["dz"], G, act)
    torch.cuda.synchronize()
    assert torch.equal(y, y2), "not bitwise reproducible"
    w1, w2 = _experts_used(p, d, G, _mfma_path(T, E, H, I, topk))
    exact = O.moe_grouped_exact(p["x"], tw.numpy(), tid.numpy(), w1, w2, activation=act)
    _check(y.cpu().numpy(), exact, f"T={T} E={E} H={H} I={I} k={topk} G={G} zp={zp} {act}")


@pytest.mark.parametrize("T", [24, 512])
def test_moe_strided_rows(T):
    """Activation and output rows at strides past H (x and out as column slices of wider
    buffers), through the stream kernels (T = 24, 6 routes per expert) and the tile kernels
    (T = 512, 128 per expert): the same bits as contiguous rows, and nothing written past H."""
    E, H, I, topk, G = 16, 256, 128, 4, 64
    assert _mfma_path(T, E, H, I, topk) == (T == 512)
    p, d = _problem(T, E, H, I, topk, G, True, seed=T + 7)
    tw, tid = _route_cpu(torch.from_numpy(p["logits"]), topk)
    tw, tid = tw.to(DEV), tid.to(DEV)
    x = _dev(p["x"])
    args = (d["gq"], d["gs"], d["gz"], d["dq"], d["ds"], d["dz"], G)
    y = ops.moe(x, tw, tid, *args)
    xb = torch.zeros((T, H + 64), dtype=x.dtype, device=DEV)
    xb[:, :H] = x
    ob = torch.full((T, H + 32), 7.0, dtype=x.dtype, device=DEV)
    ys = ops.moe(xb[:, :H], tw, tid, *args, out=ob[:, :H])
    torch.cuda.synchronize()
    assert ys.data_ptr() == ob.data_ptr()
    assert torch.equal(ys, y)
    assert bool((ob[:, H:] == 7.0).all())


def test_moe_skewed_routing_multiple_passes():
    # every route on two experts: 600 rows per expert -> several wave-group passes
    T, E, H, I, topk, G = 600, 8, 256, 128, 2, 128
    p, d = _problem(T, E, H, I, topk, G, seed=5)
    tid = torch.tensor([[3, 6]] * T, dtype=torch.int64)
    tw = torch.rand(T, topk, generator=torch.Generator().manual_seed(0))
    y = ops.moe(_dev(p["x"]), tw.to(DEV), tid.to(DEV), d["gq"], d["gs"], d["gz"], d["dq"], d["ds"], d["dz"], G)
    w1, w2 = _experts_used(p, d, G, _mfma_path(T, E, H, I, topk))
    exact = O.moe_grouped_exact(p["x"], tw.numpy(), tid.numpy(), w1, w2)
    _check(y.cpu().numpy(), exact, "skewed")


def test_moe_bf16_activations_and_out_of_range_ids():
    T, E, H, I, topk, G = 20, 8, 256, 128, 3, 64
    p, d = _problem(T, E, H, I, topk, G, seed=6)
    tw, tid = _route_cpu(torch.from_numpy(p["logits"]), topk)
    tid = tid.clone()
    tid[::4, 1] = E + 3  # ignored routes
    xb = torch.from_numpy(p["x"]).float().bfloat16()
    y = ops.moe(xb.to(DEV), tw.to(DEV), tid.to(DEV), d["gq"], d["gs"], d["gz"], d["dq"], d["ds"], d["dz"], G)
    # bf16 activations, 7.5 routes per expert (the decode-structured kernels): unrounded weights
    assert not _mfma_path(T, E, H, I, topk)
    w1b, w2b = _unrounded_experts(p, G)
    xf = xb.float().numpy()
    exact = O.moe_grouped_exact(xf, tw.numpy(), tid.numpy(), w1b, w2b, inter_dtype="bfloat16")
    yf = y.float().cpu().numpy()
    floor = float(np.sqrt(np.mean(exact ** 2)))
    d_ = np.abs(yf - exact)
    # bf16 output: one bf16 ulp is 8 fp16 ulps
    assert np.max(d_ / O.fp16_ulp(exact, floor)) <= 16.0
    assert d_.sum() / np.abs(exact).sum() <= 2e-3


def test_moe_tokens_without_routes_get_zero_rows():
    """Tokens none of whose ids is in [0, E) (expert parallelism: every expert elsewhere) sum
    nothing: their output rows are zero, with the stream kernels (few routes per expert) and
    the grouped tile kernels (many)."""
    for T, E in ((12, 16), (600, 8)):
        H, I, topk, G = 256, 128, 4 if E == 16 else 2, 64
        p, d = _problem(T, E, H, I, topk, G, seed=11)
        tw, tid = _route_cpu(torch.from_numpy(p["logits"]), topk)
        tid = tid.clone()
        tid[2] = -1          # all routes masked (negative ids)
        tid[5] = E + 1       # all routes masked (ids past the experts)
        tid[7, 1:] = -1      # one route left
        out = torch.full((T, H), float("nan"), dtype=torch.float16, device=DEV)
        y = ops.moe(_dev(p["x"]), tw.to(DEV), tid.to(DEV), d["gq"], d["gs"], d["gz"], d["dq"], d["ds"], d["dz"], G,
                    out=out)
        torch.cuda.synchronize()
        yc = y.cpu()
        assert not torch.isnan(yc).any(), (T, E)
        assert torch.equal(yc[2], torch.zeros(H, dtype=torch.float16)), (T, E)
        assert torch.equal(yc[5], torch.zeros(H, dtype=torch.float16)), (T, E)
        w1, w2 = _experts_used(p, d, G, _mfma_path(T, E, H, I, topk, G))
        exact = O.moe_grouped_exact(p["x"], tw.numpy(), tid.numpy(), w1, w2)
        keep = np.ones(T, dtype=bool)
        keep[[2, 5]] = False
        _check(yc.numpy()[keep], exact[keep], f"masked tokens T={T} E={E}")


def test_gemma4_grouped_surface_ref_layout_with_zeros():
    T, E, H, I, topk, G = 24, 8, 256, 256, 2, 32
    p, d = _problem(T, E, H, I, topk, G, seed=7)
    tw, tid = _route_cpu(torch.from_numpy(p["logits"]), topk)
    gq, gz, gs = p["gate_up"]
    dq, dz, ds = p["down"]
    ref_gu = [O.repack_awq_to_ref(gq[e], gz[e], gs[e]) for e in range(E)]
    ref_dn = [O.repack_awq_to_ref(dq[e], dz[e], ds[e]) for e in range(E)]
    stack = lambda lst, i: _dev(np.stack([t[i] for t in lst]))
    out, used, reason = MOE.gemma4_moe_int4_prefill_grouped(
        _dev(p["x"]), tw.to(DEV), tid.to(DEV), stack(ref_gu, 0), stack(ref_gu, 2), stack(ref_dn, 0),
        stack(ref_dn, 2), intermediate_dim=I, gate_up_qzeros=stack(ref_gu, 1), down_qzeros=stack(ref_dn, 1))
    assert used and reason == "ok", reason
    y_awq = ops.moe(_dev(p["x"]), tw.to(DEV), tid.to(DEV), d["gq"], d["gs"], d["gz"], d["dq"], d["ds"], d["dz"], G)
    assert torch.equal(out, y_awq)  # the repacked reference layout gives the same bits
    out2, used2, reason2 = MOE.gemma4_moe_int4_prefill_grouped(
        _dev(p["x"]), tw.to(DEV), tid.to(DEV), stack(ref_gu, 0), stack(ref_gu, 2), stack(ref_dn, 0),
        stack(ref_dn, 2), intermediate_dim=I, block_i_override=48)
    assert not used2 and reason2 == "invalid_prefill_grouped_tile"


def _route_logits_spec(logits16: np.ndarray, topk: int):
    """fused_moe's routing flow (fused_moe.py:12-15) on 16-bit logits, specified exactly:
    probabilities = the softmax correctly rounded to fp16 (float64 exp and sum), the top-k by
    probability with equal ones in ascending expert id, renormalised with torch's fp16
    arithmetic: s = fp16(fp32 sum of the selected, slot order), w = fp16(fp32(p) / fp32(s)).
    Returns (p [T, E] fp16, ids [T, k], w [T, k] fp16)."""
    x = logits16.astype(np.float64)
    e = np.exp(x - x.max(-1, keepdims=True))
    p = (e / e.sum(-1, keepdims=True)).astype(np.float16)
    T, E = p.shape
    order = np.lexsort((np.broadcast_to(np.arange(E), (T, E)), -p.astype(np.float64)), axis=-1)
    ids = order[:, :topk]
    sel = np.take_along_axis(p, ids, 1)
    s = np.zeros(T, dtype=np.float32)
    for j in range(topk):
        s = (s + sel[:, j].astype(np.float32)).astype(np.float32)
    w = (sel.astype(np.float32) / s.astype(np.float16).astype(np.float32)[:, None]).astype(np.float16)
    return p, ids, w


def _unambiguous(p16_port: np.ndarray, p16_spec: np.ndarray, topk: int) -> np.ndarray:
    """Tokens whose port probabilities equal the specification's and hold no ties among the
    top k + 1 (torch.topk leaves the order of equal values open, so only these tokens have one
    right answer for the ids)."""
    same = (p16_port.view(np.uint16) == p16_spec.view(np.uint16)).all(-1)
    top = -np.sort(-p16_spec.astype(np.float64), axis=-1)[:, : topk + 1]
    distinct = (np.diff(top, axis=-1) != 0).all(-1)
    return same & distinct


@pytest.mark.parametrize("T", [16, 512])
def test_fused_moe_routing_ids_match_port(T):
    """configs[4] logits (E=64, top-8, fp16) through fused_moe's dtype flow on the device: ids
    and fp16 weights equal the exact specification bit for bit on every token, and equal the
    port (torch CPU softmax -> topk -> renormalise, oracle.ref_cpu.moe_routing_cpu) bit for bit
    on every token where the port's answer is unique (no ties among the top 9, probabilities
    rounded alike); elsewhere the device's choice is a valid top-8 of the port's probabilities."""
    E, topk = 64, 8
    p = make_moe_problem(T, E=E, top_k=topk, H=64, I=64, group_size=32, seed=40 + T)
    logits = p["logits"]
    w, ids = ops.moe_route(_dev(logits), topk, flow="logits")
    assert w.dtype == torch.float16 and ids.dtype == torch.int32
    w, ids = w.cpu().numpy(), ids.cpu().numpy()
    p_spec, ids_spec, w_spec = _route_logits_spec(logits, topk)
    assert np.array_equal(ids, ids_spec)
    assert np.array_equal(w.view(np.uint16), w_spec.view(np.uint16))
    lt = torch.from_numpy(logits)
    p_port = torch.softmax(lt, dim=-1).numpy()
    tw_port, tid_port = R.moe_routing_cpu(lt, topk)
    ok = _unambiguous(p_port, p_spec, topk)
    print(f"T={T}: {int(ok.sum())} of {T} tokens unambiguous", flush=True)
    assert ok.mean() >= 0.9
    assert np.array_equal(ids[ok], tid_port.numpy()[ok])
    assert np.array_equal(w[ok].view(np.uint16), tw_port.numpy()[ok].view(np.uint16))
    for t in np.nonzero(~ok)[0]:
        chosen = p_port[t, ids[t]].astype(np.float64)
        rest = np.delete(p_port[t].astype(np.float64), ids[t])
        assert chosen.min() >= rest.max() - O.fp16_ulp(np.array([rest.max()]), floor=2.0 ** -24)[0]


@pytest.mark.parametrize("T", [16, 512])
def test_gemma4_router_flow(T):
    """The Gemma4 router's flow (models/gemma4/moe.py:106-123): fp32 softmax, top-8, w / max(sum,
    1e-8) in fp32, then cast to the hidden dtype.  Ids equal torch's on every token whose top 9
    fp32 probabilities are distinct (ties: lower id first); fp16 weights within one ulp of the
    cast of torch's fp32 weights, nearly all bit-equal."""
    E, topk = 64, 8
    p = make_moe_problem(T, E=E, top_k=topk, H=64, I=64, group_size=32, seed=41 + T)
    lt = torch.from_numpy(p["logits"])
    w, ids = ops.moe_route(lt.to(DEV), topk, flow="fp32", weights_dtype=torch.float16)
    assert w.dtype == torch.float16
    pf = torch.softmax(lt.float(), dim=-1)
    tw, _ = torch.topk(pf, topk, dim=-1)
    order = np.lexsort((np.broadcast_to(np.arange(E), (T, E)), -pf.double().numpy()), axis=-1)
    tid = torch.from_numpy(order[:, :topk])
    tw = torch.take_along_dim(pf, tid, 1)
    want = (tw / tw.sum(-1, keepdim=True).clamp_min(1e-8)).half().numpy()
    top = -np.sort(-pf.double().numpy(), axis=-1)[:, : topk + 1]
    distinct = (np.diff(top, axis=-1) < -1e-6 * top[:, 1:]).all(-1)
    assert distinct.mean() >= 0.9
    got_ids = ids.cpu().numpy()
    assert np.array_equal(got_ids[distinct], tid.numpy()[distinct])
    got = w.cpu().numpy()
    d = np.abs(got[distinct].astype(np.float64) - want[distinct].astype(np.float64))
    assert (d <= O.fp16_ulp(want[distinct].astype(np.float64), floor=2.0 ** -24)).all()
    assert (got[distinct].view(np.uint16) == want[distinct].view(np.uint16)).mean() >= 0.99


def test_fused_moe_surface_against_reference_port():
    T, E, H, I, topk, G = 40, 16, 256, 128, 4, 64
    p, d = _problem(T, E, H, I, topk, G, seed=8)
    logits = torch.from_numpy(p["logits"])
    w1 = MOE.AWQExperts(d["gq"], d["gs"], d["gz"], G, layout="autoawq")
    w2 = MOE.AWQExperts(d["dq"], d["ds"], d["dz"], G, layout="autoawq")
    y = MOE.fused_moe(_dev(p["x"]), w1, w2, logits.to(DEV), topk).cpu()
    # the routes the surface took: fused_moe's dtype flow, pinned above against the port
    tw, tid = ops.moe_route(logits.to(DEV), topk, flow="logits")
    tw, tid = tw.cpu(), tid.cpu().long()
    w1d, w2d = _dense_experts(d, G)
    port = R.fused_moe_cpu(torch.from_numpy(p["x"]), torch.from_numpy(w1d), torch.from_numpy(w2d),
                           topk_weights=tw, topk_ids=tid).double().numpy()
    w1u, w2u = _experts_used(p, d, G, _mfma_path(T, E, H, I, topk))
    exact = O.moe_grouped_exact(p["x"], tw.float().numpy(), tid.numpy(), w1u, w2u)
    _check(y.numpy(), exact, "fused_moe")
    floor = float(np.sqrt(np.mean(exact ** 2)))
    # the port's fp16 intermediates and accumulation: a few ulps from both
    assert np.max(np.abs(y.double().numpy() - port) / O.fp16_ulp(exact, floor)) <= 10.0


@pytest.mark.parametrize("T", [16, 512])
def test_config4_full_size(T):
    """BASELINE config 4 at its real shape: E=64, top-8, H=2048, I=1024, g=128, zero points."""
    E, H, I, topk, G = 64, 2048, 1024, 8, 128
    p, d = _problem(T, E, H, I, topk, G, seed=40 + T)
    tw, tid = _route_cpu(torch.from_numpy(p["logits"]), topk)
    y = ops.moe(_dev(p["x"]), tw.to(DEV), tid.to(DEV), d["gq"], d["gs"], d["gz"], d["dq"], d["ds"], d["dz"], G)
    w1, w2 = _experts_used(p, d, G, _mfma_path(T, E, H, I, topk))
    exact = O.moe_grouped_exact(p["x"], tw.numpy(), tid.numpy(), w1, w2)
    _check(y.cpu().numpy(), exact, f"config4 T={T}")


@pytest.mark.parametrize("T", [16, 512])
def test_config4_full_size_vs_fused_moe_port(T):
    """configs[4] at its real shape (E=64, top-8, H=2048, I=1024, g=128, zero points) through
    the ``fused_moe`` surface against the port of the reference's own path (dequantized fp16
    experts, ``fused_moe_cpu``: fp16 GEMMs, fp16 intermediates and fp16 accumulation, the
    serialized per-token branch at T = 512, fused_moe.py:21, 57-75) on the same routes.

    Bar, absolute and in ulps: |y - port| <= 12 fp16 ulps at max(|port|, RMS) and mean relative
    error <= 1e-3, the north star's mean-relative bar.  The port itself sits up to 0.58 absolute (6.3 ulps at the RMS scale, RMS
    42-50) and 7e-4 mean relative from the exact result (float64, measured on the CPU for these
    seeds); the kernel sits within 4 ulps of it (test_config4_full_size).  The north star's 2e-2
    absolute bar is below one fp16 ulp (0.03-0.06) at this output magnitude, so it cannot hold
    for any fp16 output, the reference's included."""
    E, H, I, topk, G = 64, 2048, 1024, 8, 128
    p, d = _problem(T, E, H, I, topk, G, seed=40 + T)
    logits = _dev(p["logits"])
    w1 = MOE.AWQExperts(d["gq"], d["gs"], d["gz"], G, layout="autoawq")
    w2 = MOE.AWQExperts(d["dq"], d["ds"], d["dz"], G, layout="autoawq")
    print(f"config4 fused_moe T={T}", flush=True)
    y = MOE.fused_moe(_dev(p["x"]), w1, w2, logits, topk).double().cpu().numpy()
    tw, tid = ops.moe_route(logits, topk, flow="logits")
    w1d, w2d = _dense_experts(d, G)
    port = R.fused_moe_cpu(torch.from_numpy(p["x"]), torch.from_numpy(w1d), torch.from_numpy(w2d),
                           topk_weights=tw.cpu(), topk_ids=tid.cpu().long()).double().numpy()
    rms = float(np.sqrt(np.mean(port ** 2)))
    d_ = np.abs(y - port)
    ulps = d_ / O.fp16_ulp(port, rms)
    mrel = float(d_.sum() / np.abs(port).sum())
    print(f"config4 T={T} vs port: max abs {d_.max():.4f}, max ulp@max(|y|,rms) {ulps.max():.2f}, "
          f"mean rel {mrel:.2e}, rms {rms:.1f}", flush=True)
    assert ulps.max() <= 12.0 and mrel <= 1e-3


def test_moe_mfma_path_bf16():
    T, E, H, I, topk, G = 96, 4, 256, 128, 2, 64   # 48 routes per expert
    p, d = _problem(T, E, H, I, topk, G, seed=9)
    tw, tid = _route_cpu(torch.from_numpy(p["logits"]), topk)
    xb = torch.from_numpy(p["x"]).float().bfloat16()
    y = ops.moe(xb.to(DEV), tw.to(DEV), tid.to(DEV), d["gq"], d["gs"], d["gz"], d["dq"], d["ds"], d["dz"], G)
    gq, gz, gs = p["gate_up"]
    dq, dz, ds = p["down"]
    bf = lambda q, s, z: O.bf16_bits_to_f32(O.dequant_awq(q, s, z, G, out_dtype="bfloat16")).T
    w1b = np.stack([bf(gq[e], gs[e], gz[e]) for e in range(E)])
    w2b = np.stack([bf(dq[e], ds[e], dz[e]) for e in range(E)])
    exact = O.moe_grouped_exact(xb.float().numpy(), tw.numpy(), tid.numpy(), w1b, w2b, inter_dtype="bfloat16")
    yf = y.float().cpu().numpy()
    floor = float(np.sqrt(np.mean(exact ** 2)))
    d_ = np.abs(yf - exact)
    assert np.max(d_ / O.fp16_ulp(exact, floor)) <= 16.0
    assert d_.sum() / np.abs(exact).sum() <= 2e-3



@pytest.mark.parametrize("wdtype", [torch.float16, torch.bfloat16])
def test_moe_mfma_path_16bit_routing_weights(wdtype):
    # the tile kernels read fp32 routing weights by LDS DMA and 16-bit ones by plain loads:
    # the same weight values in either dtype give the same bits
    T, E, H, I, topk, G = 96, 4, 256, 128, 2, 64   # 48 routes per expert: tile kernels
    p, d = _problem(T, E, H, I, topk, G, seed=11)
    tw, tid = _route_cpu(torch.from_numpy(p["logits"]), topk)
    tw16 = tw.to(wdtype)
    x = _dev(p["x"])
    args = (d["gq"], d["gs"], d["gz"], d["dq"], d["ds"], d["dz"], G)
    y16 = ops.moe(x, tw16.to(DEV), tid.to(DEV), *args)
    y32 = ops.moe(x, tw16.float().to(DEV), tid.to(DEV), *args)
    torch.cuda.synchronize()
    assert torch.equal(y16.view(torch.int16), y32.view(torch.int16))


def test_moe_tile_path_experts_past_64_skewed():
    """E = 128 on the tile path with the routes skewed onto experts 64 and above: experts 70 and
    100 take 200 routes each (two full 96-route tiles and a partial one), experts 64 .. 127 the
    rest, experts 0 .. 63 none, so every row tile belongs to the tile search's second pass of
    64 experts (full tiles first, then the partial ones)."""
    T, E, H, I, topk, G = 512, 128, 256, 128, 4, 64
    assert _mfma_path(T, E, H, I, topk, G)
    p, d = _problem(T, E, H, I, topk, G, seed=17)
    g = torch.Generator().manual_seed(17)
    tid = torch.empty((T, topk), dtype=torch.int64)
    tid[:, 0] = torch.where(torch.arange(T) < 200, 70, 64 + torch.randint(0, 64, (T,), generator=g))
    tid[:, 1] = torch.where(torch.arange(T) >= T - 200, 100, 64 + torch.randint(0, 64, (T,), generator=g))
    tid[:, 2:] = 64 + torch.randint(0, 64, (T, topk - 2), generator=g)
    # distinct experts per token (a token's routes to one expert would be summed twice anyway,
    # but keep the reference's top-k shape)
    for t in range(T):
        seen = set()
        for j in range(topk):
            e = int(tid[t, j])
            while e in seen:
                e = 64 + (e - 64 + 1) % 64
            tid[t, j] = e
            seen.add(e)
    tw = torch.rand(T, topk, generator=g)
    counts = torch.bincount(tid.flatten(), minlength=E)
    assert int(counts[:64].sum()) == 0 and int(counts[70]) >= 192 and int(counts[100]) >= 192
    y = ops.moe(_dev(p["x"]), tw.to(DEV), tid.to(DEV), d["gq"], d["gs"], d["gz"], d["dq"], d["ds"], d["dz"], G)
    w1, w2 = _experts_used(p, d, G, True)
    exact = O.moe_grouped_exact(p["x"], tw.numpy(), tid.numpy(), w1, w2)
    _check(y.cpu().numpy(), exact, "E=128 skewed onto experts 64..127")


def test_moe_tile_path_out_of_range_ids():
    # ids outside [0, E) on the tile path (32 routes per expert): the route lists leave them
    # out and the combine adds nothing for them
    T, E, H, I, topk, G = 128, 8, 256, 128, 2, 64
    assert _mfma_path(T, E, H, I, topk, G)
    p, d = _problem(T, E, H, I, topk, G, seed=19)
    tw, tid = _route_cpu(torch.from_numpy(p["logits"]), topk)
    tid = tid.clone()
    tid[::5, 1] = E + 3
    tid[2::7, 0] = -1
    y = ops.moe(_dev(p["x"]), tw.to(DEV), tid.to(DEV), d["gq"], d["gs"], d["gz"], d["dq"], d["ds"], d["dz"], G)
    w1, w2 = _experts_used(p, d, G, True)
    exact = O.moe_grouped_exact(p["x"], tw.numpy(), tid.numpy(), w1, w2)
    _check(y.cpu().numpy(), exact, "tile path, ids outside [0, E)")


def test_moe_tile_path_fewer_row_tiles_than_experts():
    # every route on experts 5 and 2 (256 each: two full 96-route tiles and a 64-route
    # partial per expert, six row tiles for eight experts): row tile t is not expert t's, and
    # the blocks of row tiles 6 and 7 find no tile at all
    T, E, H, I, topk, G = 256, 8, 256, 128, 2, 128
    assert _mfma_path(T, E, H, I, topk, G)
    p, d = _problem(T, E, H, I, topk, G, seed=13)
    tid = torch.tensor([[5, 2]] * T, dtype=torch.int64)
    tw = torch.rand(T, topk, generator=torch.Generator().manual_seed(1))
    y = ops.moe(_dev(p["x"]), tw.to(DEV), tid.to(DEV), d["gq"], d["gs"], d["gz"], d["dq"], d["ds"], d["dz"], G)
    w1, w2 = _experts_used(p, d, G, True)
    exact = O.moe_grouped_exact(p["x"], tw.numpy(), tid.numpy(), w1, w2)
    _check(y.cpu().numpy(), exact, "fewer row tiles than experts")


@pytest.mark.parametrize("T", [12, 200])
@pytest.mark.parametrize("form", ["dense_gated", "dense_ungated", "awq_ungated"])
def test_fused_moe_dense_and_ungated_forms(T, form):
    """``fused_moe`` with dense expert tensors (the materialised experts the reference's zero-point
    Gemma4 path hands over, gemma4/moe.py:722-750, 788) and with an ungated ``w1`` of I rows
    (fused_moe.py:52-53; an AWQ stack is dequantized by the HIP kernel first): the reference's own
    expert loop, grouped by expert at T = 12 and token by token at T = 200 (M > 128,
    fused_moe.py:21), against the port on the same routes.  fp16 sums in a different order (the
    device's index_add_ is unordered, and the device GEMMs accumulate in their own order): within
    10 fp16 ulps at max(|y|, RMS), as the kernel-vs-port bar above, and mean relative 1e-3."""
    E, H, I, topk, G = 8, 256, 128, 2, 64
    print(f"fused_moe {form} T={T}", flush=True)
    p, d = _problem(T, E, H, I, topk, G, seed=50 + T)
    logits = _dev(p["logits"])
    w1d, w2d = _dense_experts(d, G)
    x = _dev(p["x"])
    if form == "dense_gated":
        w1, w2, w1p = torch.from_numpy(w1d).to(DEV), torch.from_numpy(w2d).to(DEV), w1d
    elif form == "dense_ungated":
        w1, w2, w1p = torch.from_numpy(w1d[:, :I]).to(DEV), torch.from_numpy(w2d).to(DEV), w1d[:, :I]
    else:
        w1 = MOE.AWQExperts(d["gq"][:, :, : I // 8].contiguous(), d["gs"][:, :, :I].contiguous(),
                            d["gz"][:, :, : I // 8].contiguous(), G, layout="autoawq")
        w2 = MOE.AWQExperts(d["dq"], d["ds"], d["dz"], G, layout="autoawq")
        w1p = w1d[:, :I]
    y = MOE.fused_moe(x, w1, w2, logits, topk).double().cpu().numpy()
    tw, tid = ops.moe_route(logits, topk, flow="logits")
    port = R.fused_moe_cpu(torch.from_numpy(p["x"]), torch.from_numpy(np.ascontiguousarray(w1p)),
                           torch.from_numpy(w2d), topk_weights=tw.cpu(), topk_ids=tid.cpu().long()).double().numpy()
    rms = float(np.sqrt(np.mean(port ** 2)))
    d_ = np.abs(y - port)
    print(f"  max ulp {(d_ / O.fp16_ulp(port, rms)).max():.2f}, mean rel {d_.sum() / np.abs(port).sum():.2e}", flush=True)
    assert (d_ / O.fp16_ulp(port, rms)).max() <= 10.0
    assert d_.sum() / np.abs(port).sum() <= 1e-3
    if form == "awq_ungated":  # the dequantized stacks are held by the AWQ tensors, not rebuilt
        held = ops.derived_copies(w1.qweight)
        assert "moe_dense_experts" in held and tuple(held["moe_dense_experts"].shape) == (E, I, H)


def test_fused_moe_rejects_mixed_and_misshaped_experts():
    E, H, I, topk, G = 4, 128, 64, 2, 32
    p, d = _problem(4, E, H, I, topk, G, seed=3)
    w1 = MOE.AWQExperts(d["gq"], d["gs"], d["gz"], G, layout="autoawq")
    dense = torch.zeros((E, H, I), dtype=torch.float16, device=DEV)
    with pytest.raises(TypeError):
        MOE.fused_moe(_dev(p["x"]), w1, dense, _dev(p["logits"]), topk)
    with pytest.raises(ValueError):
        MOE.fused_moe(_dev(p["x"]), torch.zeros((E, 3 * I, H), dtype=torch.float16, device=DEV), dense,
                      _dev(p["logits"]), topk)
