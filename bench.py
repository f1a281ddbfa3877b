"""Benchmark of the AWQ W4A16 hot path on one MI355X.

Workload (``config.workload``): the decode GEMV sweep of the benchmark configuration
(configs[1]): M in {1, 4, 16}, K = 4096, N in {4096, 6144, 24576}, group 128, AutoAWQ
packing, fp16 activations.  One *step* = the nine GEMMs once, each on its own weight
copy; steps rotate over enough copies (>= 1 GiB) that weights are read from HBM, not from
the 256 MB Infinity Cache.  The whole step is captured once in a HIP graph and replayed, so
host launch overhead is not timed.

``value`` = algorithmic bytes of one step (weights + scales + zeros + x + y, no split-K
scratch, no re-reads) x steps / elapsed time, in GB/s.

Extra measurements on the same JSON line:
  * ``roofline``: the decode kernel at M=1, N=24576 (the heaviest single launch and the
    headline M=1 target) -- algorithmic bytes per launch / average launch duration from HIP
    events around back-to-back launches on the launch stream, against 8 TB/s;
  * ``prefill``: configs[3] at M=2048, N=24576 in TFLOP/s against 2.5 PFLOP/s dense fp16;
  * ``moe``: configs[4] (E=64, top-8, H=2048, I=1024, g=128) at T=16 and T=512: routing +
    grouped gate_up/activation/down + combine per step, algorithmic bytes (distinct experts
    touched x expert bytes + x + y) against 8 TB/s and flops against 2.5 PFLOP/s;
  * ``cpu_baseline``: the reference's CPU path (dequant + F.linear, restated in
    ``oracle/ref_cpu.py``) on a bounded sample of the same sweep, timed on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
K_DEC, G = 4096, 128
SWEEP = [(m, n) for m in (1, 4, 16) for n in (4096, 6144, 24576)]


def alg_bytes(M, K, N, g=G):
    return K * N // 2 + (K // g) * N * 2 + (K // g) * (N // 8) * 4 + M * K * 2 + M * N * 2


def _weights(torch, K, N, copies, dev, seed):
    """`copies` independent AutoAWQ-packed weight sets, generated on the device with the
    benchmark distributions (int4 uniform, zeros uniform, scales |N(0,.02)|+1e-4)."""
    gen = torch.Generator(device=dev).manual_seed(seed)
    out = []
    for _ in range(copies):
        qw = torch.randint(-2**31, 2**31 - 1, (K, N // 8), dtype=torch.int32, device=dev, generator=gen)
        qz = torch.randint(-2**31, 2**31 - 1, (K // G, N // 8), dtype=torch.int32, device=dev, generator=gen)
        sc = (torch.randn((K // G, N), device=dev, generator=gen).abs() * 0.02 + 1e-4).half()
        out.append((qw, qz, sc))
    return out


def _progress(what):
    """One line per bench leg on stderr (stdout carries only the JSON result)."""
    print(f"[bench] {what}", file=sys.stderr, flush=True)


_SIDE_STREAM = []


def _side_stream(torch):
    """One side stream for the warm-ups of every measurement, the graphs captured on torch's own
    capture stream.  Measured on MI355X (M = 1, N = 24576, graph of 210 launches): replays run
    11.0 us per launch this way in every measurement of a run; with a new warm-up stream per
    measurement every measurement after the first ran 12.2 us, and so did graphs captured on
    the warm-up stream itself or warmed up on the default stream."""
    if not _SIDE_STREAM:
        _SIDE_STREAM.append(torch.cuda.Stream())
    return _SIDE_STREAM[0]


def _time_graph(torch, fn, reps, warmup=3):
    """Capture fn() in a HIP graph, replay `reps` times between events; returns ms/replay."""
    s = _side_stream(torch)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warmup):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):  # torch's capture stream, not the warm-up stream (see _side_stream)
        fn()
    g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / reps, g


def _cpu_host():
    """Host CPU facts for the CPU baseline: os.cpu_count(), the cores this process may run on
    (affinity), the cgroup CPU quota, the model name (lscpu), and the thread count used: all
    cores (os.cpu_count()), or fewer when the affinity mask or the quota allows fewer."""
    import subprocess
    count = os.cpu_count() or 1
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else count
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
            if q != "max":
                quota = max(1, int(int(q) // int(period)))
    except (OSError, ValueError):
        pass
    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        model = next((l.split(":", 1)[1].strip() for l in out.splitlines() if l.startswith("Model name")), None)
    except (OSError, subprocess.SubprocessError):
        pass
    threads = min(c for c in (count, affinity, quota) if c)
    return {"os_cpu_count": count, "affinity_cores": affinity, "cgroup_quota_cpus": quota,
            "model": model, "threads": threads}


def _median_time(fn, reps):
    """Median wall time of fn() over `reps` calls after one warm-up call."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2]


def cpu_baseline(reps=5):
    """The reference's CPU path restated (oracle/ref_cpu.py), timed on the host cores with
    torch.set_num_threads(all cores), median of `reps` after one warm-up, per configuration:
      * cold = dequant (int64 shifts, fp32 math, tensor.py:835-860) + F.linear in fp16 per
        call; warm = F.linear on the cached fp16 weight only (the reference's LRU steady
        state, tensor.py:1125-1129, 1142);
      * configs[1] (the headline: the nine decode shapes, algorithmic GB/s), configs[0],
        configs[2] (M in {1, 8, 32}; split-K is a GPU knob), configs[3] on a 64-row sample of
        M = 2048 (TFLOP/s), configs[4] through the restated fused_moe over dense fp16 experts
        (T = 16 grouped branch; T = 512 serialized per-token branch, fused_moe.py:21, on a
        64-token sample scaled to 512; cold adds the dequantization of the experts touched).
    Returns the cpu_baseline object (value = configs[1] cold GB/s) with the per-config legs."""
    import numpy as np
    import torch
    from oracle import ref_cpu as R

    host = _cpu_host()
    torch.set_num_threads(host["threads"])
    rng = np.random.default_rng(0)
    t_start = time.perf_counter()

    def ref_weight(K, N):
        qw = torch.from_numpy(rng.integers(-2**31, 2**31 - 1, size=(N, K // 8), dtype=np.int64).astype(np.int32))
        qz = torch.from_numpy(rng.integers(-2**31, 2**31 - 1, size=(N, K // G // 8), dtype=np.int64).astype(np.int32))
        sc = torch.from_numpy((np.abs(rng.standard_normal((N, K // G))) * 0.02 + 1e-4).astype(np.float16))
        return qw, sc, qz  # awq_linear_cpu argument order

    def x_of(M, K):
        return torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16))

    def cold_warm(M, K, N, wts):
        x = x_of(M, K)
        cold = _median_time(lambda: R.awq_linear_cpu(x, *wts, G), reps)
        dense = R.dequantize_awq_cpu(*wts, G)
        warm = _median_time(lambda: R.awq_linear_cpu(x, *wts, G, dense_weight=dense), reps)
        return cold, warm

    legs = {}
    # the headline sweep
    W1 = {n: ref_weight(K_DEC, n) for n in (4096, 6144, 24576)}
    per = {}
    tc = tw = 0.0
    for M, N in SWEEP:
        c, w = cold_warm(M, K_DEC, N, W1[N])
        per[f"M{M}_N{N}"] = {"cold_ms": round(c * 1e3, 3), "warm_ms": round(w * 1e3, 3)}
        tc += c
        tw += w
    step = sum(alg_bytes(m, K_DEC, n) for m, n in SWEEP)
    legs["config1"] = {"cold_GBps": round(step / tc / 1e9, 4), "warm_GBps": round(step / tw / 1e9, 4),
                       "per_shape": per}
    del W1
    # configs[0]
    c, w = cold_warm(1, 2048, 5632, ref_weight(2048, 5632))
    legs["config0"] = {"M": 1, "K": 2048, "N": 5632, "cold_ms": round(c * 1e3, 3), "warm_ms": round(w * 1e3, 3),
                       "cold_GBps": round(alg_bytes(1, 2048, 5632) / c / 1e9, 4),
                       "warm_GBps": round(alg_bytes(1, 2048, 5632) / w / 1e9, 4)}
    # configs[2]
    W2 = ref_weight(12288, 4096)
    legs["config2"] = {}
    for M in (1, 8, 32):
        c, w = cold_warm(M, 12288, 4096, W2)
        legs["config2"][f"M{M}"] = {"cold_ms": round(c * 1e3, 3), "warm_ms": round(w * 1e3, 3)}
    del W2
    # 64 of the 2048 rows
    rows, K3, N3 = 64, K_DEC, 24576
    c, w = cold_warm(rows, K3, N3, ref_weight(K3, N3))
    fl = 2.0 * rows * K3 * N3
    legs["config3"] = {"sample": f"{rows} rows of M=2048, K={K3}, N={N3}", "cold_ms": round(c * 1e3, 2),
                       "warm_ms": round(w * 1e3, 2), "cold_TFLOPs": round(fl / c / 1e12, 5),
                       "warm_TFLOPs": round(fl / w / 1e12, 5)}
    # fused_moe over dense fp16 experts (distinct storage per expert)
    E, H, I, topk = MOE_E, MOE_H, MOE_I, MOE_TOPK
    w1 = torch.empty((E, 2 * I, H), dtype=torch.float16)
    w2 = torch.empty((E, H, I), dtype=torch.float16)
    w1.copy_(torch.randn((1, 2 * I, H)).mul_(0.02).half().expand(E, -1, -1))
    w2.copy_(torch.randn((1, H, I)).mul_(0.02).half().expand(E, -1, -1))
    expert_wts = [ref_weight(H, 2 * I), ref_weight(I, H)]
    deq_one = _median_time(lambda: [R.dequantize_awq_cpu(*wt, G) for wt in expert_wts], 3)
    legs["config4"] = {}
    for T, sample in ((16, 16), (512, 64)):
        x = torch.from_numpy(rng.standard_normal((sample, H)).astype(np.float16))
        logits = torch.from_numpy(rng.standard_normal((sample, E)).astype(np.float16))
        if T == 512:  # the serialized branch for all T > 128 (fused_moe.py:21): force it on the sample
            tw_, tid_ = R.moe_routing_cpu(logits, topk)
            run = lambda: R.fused_moe_cpu(x, w1, w2, topk_weights=tw_, topk_ids=tid_, serialized=True)
        else:
            run = lambda: R.fused_moe_cpu(x, w1, w2, logits, topk)
        t_s = _median_time(run, reps) * (T / sample)
        distinct = 64 if T == 512 else int(torch.unique(R.moe_routing_cpu(logits, topk)[1]).numel())
        fl = 2.0 * T * topk * (H * 2 * I + I * H)
        legs["config4"][f"T{T}"] = {"warm_ms": round(t_s * 1e3, 2), "cold_ms": round((t_s + distinct * deq_one) * 1e3, 2),
                                    "warm_TFLOPs": round(fl / t_s / 1e12, 5),
                                    "sample": f"{sample} tokens" + (" scaled to 512 (serialized branch)" if T == 512 else "")}
    del w1, w2
    return {
        "value": legs["config1"]["cold_GBps"], "unit": "GB/s", "cores": int(torch.get_num_threads()),
        "kind": "port", "warm_value": legs["config1"]["warm_GBps"], "host": host,
        "sample": "reference CPU path restated (dequant with int64 shifts and fp32 math, F.linear in fp16), "
                  f"median of {reps} after a warm-up per shape; value = configs[1] nine-shape sweep, cold "
                  f"(dequant + matmul per call); warm_value = cached fp16 weights; {time.perf_counter() - t_start:.1f} s "
                  "of CPU work in all legs",
        "legs": legs,
    }


MOE_E, MOE_TOPK, MOE_H, MOE_I, MOE_G = 64, 8, 2048, 1024, 128


def moe_expert_bytes():
    """Algorithmic bytes of one expert: gate_up (K=H, N=2I) and down (K=I, N=H) weights,
    scales and zeros."""
    w = lambda K, N: K * N // 2 + (K // MOE_G) * N * 2 + (K // MOE_G) * (N // 8) * 4
    return w(MOE_H, 2 * MOE_I) + w(MOE_I, MOE_H)


def _moe_stacks(torch, ops, dev, copies, seed):
    """`copies` expert sets (AutoAWQ stacks with the benchmark distributions), each with its
    MoE stream copies built ahead of the timed region."""
    gen = torch.Generator(device=dev).manual_seed(seed)
    rnd = lambda *shape: torch.randint(-2**31, 2**31 - 1, shape, dtype=torch.int32, device=dev, generator=gen)
    scl = lambda *shape: (torch.randn(shape, device=dev, generator=gen).abs() * 0.02 + 1e-4).half()
    E, H, I, g = MOE_E, MOE_H, MOE_I, MOE_G
    out = []
    for _ in range(copies):
        gq, gz, gs = rnd(E, H, 2 * I // 8), rnd(E, H // g, 2 * I // 8), scl(E, H // g, 2 * I)
        dq, dz, ds = rnd(E, I, H // 8), rnd(E, I // g, H // 8), scl(E, I // g, H)
        ops.prepare_moe_stream(gq, True)
        ops.prepare_moe_stream(dq, False)
        out.append((gq, gs, gz, dq, ds, dz))
    return out


def _bench_moe(torch, ops, dev, T, copies=3, inner=4):
    """configs[4] step: routing (softmax, top-8, renormalise) + grouped gate_up/act/down +
    combine, graph-replayed over `copies` expert sets (3 x 201 MB, beyond the MALL); one graph
    passes over the sets `inner` times (12 steps), so a replay's own cost (about 20 us) is
    spread over many steps as in a model's graph."""
    gen = torch.Generator(device=dev).manual_seed(100 + T)
    stacks = _moe_stacks(torch, ops, dev, copies, 200 + T)
    x = torch.randn((T, MOE_H), device=dev, generator=gen).half()
    logits = torch.randn((T, MOE_E), device=dev, generator=gen).half()
    y = torch.empty((T, MOE_H), device=dev, dtype=torch.float16)
    _, tid = ops.moe_route(logits, MOE_TOPK)
    distinct = int(torch.unique(tid).numel())

    def run():
        for _ in range(inner):
            for st in stacks:
                tw, ids = ops.moe_route(logits, MOE_TOPK)
                ops.moe(x, tw, ids, *st, MOE_G, out=y)
    ms, g = _time_graph(torch, run, 5)
    del g, stacks
    us = ms * 1e3 / (copies * inner)
    nbytes = distinct * moe_expert_bytes() + 2 * T * MOE_H * 2
    flops = 2.0 * T * MOE_TOPK * (MOE_H * 2 * MOE_I + MOE_I * MOE_H)
    gbs = nbytes / (us * 1e-6) / 1e9
    tfl = flops / (us * 1e-6) / 1e12
    return {"T": T, "E": MOE_E, "top_k": MOE_TOPK, "H": MOE_H, "I": MOE_I, "group": MOE_G,
            "distinct_experts": distinct, "us": round(us, 2), "bytes": nbytes, "GBps": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "TFLOPs": round(tfl, 1),
            "mfma_frac": round(tfl / MFMA_F16_PEAK_TFLOPS, 4)}


def _bench_rmsnorm(torch, ops, dev, copies=24):
    """rmsnorm_awq_fused_linear's device path (norm prologue + GEMM, fp16) against the GEMM
    alone on the same rotated weights (24 x 12.6 MB, beyond the MALL), graph-replayed."""
    K, N = K_DEC, 6144
    W = _weights(torch, K, N, copies, dev, 31)
    gen = torch.Generator(device=dev).manual_seed(32)
    nw = (1 + 0.1 * torch.randn(K, device=dev, generator=gen)).half()
    out = []
    for M in (1, 16, 2048):
        x = torch.randn((M, K), device=dev, generator=gen).half()
        y = torch.empty((M, N), device=dev, dtype=torch.float16)
        ws = W if M <= 32 else W[:3]

        def fused():
            for qw, qz, sc in ws:
                ops.rmsnorm_gemm(x, nw, 1e-6, qw, sc, qz, G, layout="autoawq", out=y)

        def plain():
            for qw, qz, sc in ws:
                ops.gemm(x, qw, sc, qz, G, layout="autoawq", out=y)
        ms_f, g = _time_graph(torch, fused, 10)
        del g
        ms_p, g = _time_graph(torch, plain, 10)
        del g
        us_f, us_p = ms_f * 1e3 / len(ws), ms_p * 1e3 / len(ws)
        out.append({"M": M, "K": K, "N": N, "us_fused": round(us_f, 2), "us_gemm_only": round(us_p, 2),
                    "GBps_fused": round(alg_bytes(M, K, N) / (us_f * 1e-6) / 1e9, 1)})
    del W
    return out


def _traffic():
    """HBM bytes per launch of the roofline kernel from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, each scaled by the copy-kernel calibration), or None."""
    path = os.path.join(ROOT, "profiles", "decode_m1_k4096_n24576_traffic.json")
    try:
        with open(path) as f:
            return int(json.load(f)["hbm_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


ROT_BYTES = 1 << 30  # every timed rotation reads at least this many distinct weight bytes


def weight_bytes(K, N, g=G):
    return K * N // 2 + (K // g) * N * 2 + (K // g) * (N // 8) * 4


def rot_copies(K, N):
    """Weight copies whose rotation reads >= 1 GiB (beyond the 256 MB Infinity Cache)."""
    return max(2, -(-ROT_BYTES // weight_bytes(K, N)))


def _time_rotation(torch, ops, X, pool, Y, reps, fn=None, **kw):
    """us per launch of gemm(X, w) (or ``fn``, same arguments) over every weight copy of `pool`
    (a graph of back-to-back launches, replayed `reps` times).  The graph passes over the pool
    often enough to hold at least 200 launches: a replay costs about 20 us of its own, which
    over a 21-launch graph would add 1 us to every launch."""
    inner = max(1, -(-200 // len(pool)))
    call = fn or ops.gemm

    def run():
        for _ in range(inner):
            for qw, qz, sc in pool:
                call(X, qw, sc, qz, G, layout="autoawq", out=Y, **kw)
    ms, g = _time_graph(torch, run, reps)
    del g
    return ms * 1e3 / (inner * len(pool))


def _read_ceiling(torch, dev, nbytes, copies, reps=20):
    """The HBM read ceiling of one launch that moves ``nbytes``: ``awq_w4a16_probe_read`` (16-byte
    non-temporal loads, nothing else) over ``copies`` rotated buffers, timed like the decode
    launches (graph replays of >= 200 launches); the best of five grid shapes."""
    from litevllm_amd import _lib as L
    lib = L.load()
    bufs = [torch.empty(nbytes // 4, dtype=torch.int32, device=dev) for _ in range(copies)]
    sink = torch.zeros(64, dtype=torch.int32, device=dev)
    inner = max(1, -(-200 // copies))
    best = None
    for blocks, threads, inflight in ((192, 1024, 2), (256, 1024, 4), (512, 512, 4), (1024, 256, 4), (2048, 256, 4)):
        def run():
            st = int(torch.cuda.current_stream(dev).cuda_stream)
            for _ in range(inner):
                for b in bufs:
                    L.check("awq_w4a16_probe_read", lib.awq_w4a16_probe_read(
                        int(b.data_ptr()), nbytes, blocks, threads, inflight, int(sink.data_ptr()), st))
        ms, g = _time_graph(torch, run, reps)
        del g
        us = ms * 1e3 / (inner * copies)
        if best is None or us < best[0]:
            best = (us, f"{blocks} x {threads} threads, {inflight} loads in flight per lane")
    del bufs
    gbs = nbytes / (best[0] * 1e-6) / 1e9
    return {"bytes": nbytes, "us": round(best[0], 3), "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "grid": best[1], "copies": copies}


def _hbm_entry(us, M, K, N):
    b = alg_bytes(M, K, N)
    gbs = b / (us * 1e-6) / 1e9
    return {"us": round(us, 3), "GBps": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--no-rmsnorm", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the configs[0], [2], [3] entries")
    ap.add_argument("--only", default="", help="profile mode: 'decode-m1n24576', 'prefill', 'moe-t16', "
                    "'moe-t512', 'pureread' (the read-ceiling probe) or 'copy-64MiB' (counter calibration) launches only")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(--gpus must be 1)", file=sys.stderr)
        sys.exit(2)

    import torch
    from litevllm_amd import ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev).manual_seed(1)

    if args.only == "decode-m1n24576":
        # the roofline leg's own measurement: the same >= 1 GiB rotation, captured once and
        # replayed `steps` times, so a kernel trace of this mode sees the launches bench.py times
        W = _weights(torch, K_DEC, 24576, rot_copies(K_DEC, 24576), dev, 7)
        x = torch.randn((1, K_DEC), device=dev, generator=gen).half()
        y = torch.empty((1, 24576), device=dev, dtype=torch.float16)
        for qw, qz, sc in W:
            ops.prepare_decode_stream(qw)
        torch.cuda.synchronize()
        us = _time_rotation(torch, ops, x, W, y, args.steps)
        print(f"decode M=1 K={K_DEC} N=24576: {us:.3f} us per launch over {len(W)} copies", flush=True)
        return
    if args.only in ("moe-t16", "moe-t512"):
        T = 16 if args.only == "moe-t16" else 512
        stacks = _moe_stacks(torch, ops, dev, 3, 21)
        x = torch.randn((T, MOE_H), device=dev, generator=gen).half()
        logits = torch.randn((T, MOE_E), device=dev, generator=gen).half()
        for _ in range(args.steps):
            for st in stacks:
                tw, tid = ops.moe_route(logits, MOE_TOPK)
                ops.moe(x, tw, tid, *st, MOE_G)
        torch.cuda.synchronize()
        return
    if args.only == "pureread":
        c = _read_ceiling(torch, dev, alg_bytes(1, K_DEC, 24576) // 16 * 16, rot_copies(K_DEC, 24576), reps=args.steps)
        print(f"read ceiling: {c}", flush=True)
        return
    if args.only == "copy-64MiB":
        src = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        return
    if args.only == "prefill":
        # the prefill leg's own measurement (three weight copies, graph of >= 200 launches)
        W = _weights(torch, K_DEC, 24576, 3, dev, 9)
        x = torch.randn((2048, K_DEC), device=dev, generator=gen).half()
        y = torch.empty((2048, 24576), device=dev, dtype=torch.float16)
        us = _time_rotation(torch, ops, x, W, y, args.steps)
        print(f"prefill M=2048 K={K_DEC} N=24576: {us:.1f} us per launch over {len(W)} copies", flush=True)
        return

    # ---- configs[1] decode sweep (the metric) ----
    _progress("decode sweep")
    # one weight pool per N whose rotation alone reads >= 1 GiB; step c gives shape (m, n) its
    # own copy 3 c + (index of m), so a step reads nine distinct weights and the steps rotate
    # through >= 1 GiB before any copy comes back
    step_bytes = sum(alg_bytes(m, K_DEC, n) for m, n in SWEEP)
    wbytes_step = sum(weight_bytes(K_DEC, n) for _, n in SWEEP)
    copies = max(2, -(-ROT_BYTES // wbytes_step))
    Ms = (1, 4, 16)
    pools = {n: _weights(torch, K_DEC, n, max(rot_copies(K_DEC, n), 3 * copies), dev, 100 + n) for n in (4096, 6144, 24576)}
    for n, pool in pools.items():
        for qw, _, _ in pool:
            ops.prepare_decode_stream(qw)
    X = {m: torch.randn((m, K_DEC), device=dev, generator=gen).half() for m in Ms}
    Y = {(m, n): torch.empty((m, n), device=dev, dtype=torch.float16) for m, n in SWEEP}

    def step_fn(c):
        for m, n in SWEEP:
            qw, qz, sc = pools[n][3 * c + Ms.index(m)]
            ops.gemm(X[m], qw, sc, qz, G, layout="autoawq", out=Y[(m, n)])

    def rotation():
        for c in range(copies):
            step_fn(c)

    for _ in range(max(1, args.warmup)):
        rotation()
    torch.cuda.synchronize()
    reps = max(1, -(-args.steps // copies))
    ms_rot, graph = _time_graph(torch, rotation, reps)
    steps_timed = reps * copies
    ms_per_step = ms_rot / copies
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    del graph

    # ---- per-shape launch durations: back-to-back launches over each pool (>= 1 GiB) ----
    _progress("per-shape launches")
    per_shape = {}
    for m, n in SWEEP:
        us = _time_rotation(torch, ops, X[m], pools[n], Y[(m, n)], 20)
        per_shape[f"M{m}_N{n}"] = _hbm_entry(us, m, K_DEC, n)
        per_shape[f"M{m}_N{n}"]["copies"] = len(pools[n])
        # 8-13 MB launches sit near the fixed cost of a launch (first-load latency, block
        # hand-off, dispatch: about 3.9 us), so their GB/s figure measures latency
        per_shape[f"M{m}_N{n}"]["bound"] = "hbm" if n >= 16384 else "latency"
    r = per_shape["M1_N24576"]
    roofline = {"bound": "hbm", "achieved": r["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(r["GBps"] / HBM_PEAK_GBS, 4), "traffic": _traffic(),
                "kernel": "decode_kn_kernel (decode stream layout) M=1 K=4096 N=24576",
                "bytes_per_launch": alg_bytes(1, K_DEC, 24576), "avg_launch_us": r["us"],
                "rotation_bytes": len(pools[24576]) * weight_bytes(K_DEC, 24576)}
    ncopies = len(pools[24576])
    del pools, X, Y
    # what a launch that only reads the same bytes achieves on this part, timed the same way
    _progress("read ceiling")
    ceil = _read_ceiling(torch, dev, alg_bytes(1, K_DEC, 24576) // 16 * 16, ncopies)
    ceil["decode_over_ceiling"] = round(ceil["us"] / r["us"], 4)
    roofline["read_ceiling"] = ceil

    # ---- configs[0], configs[2] (split-K 1/4/8), configs[3] (all four shapes) ----
    _progress("configs 0, 2, 3")
    configs = None
    if not args.no_configs:
        configs = {}
        W0 = _weights(torch, 2048, 5632, rot_copies(2048, 5632), dev, 50)
        x0 = torch.randn((1, 2048), device=dev, generator=gen).half()
        y0 = torch.empty((1, 5632), device=dev, dtype=torch.float16)
        configs["config0"] = _hbm_entry(_time_rotation(torch, ops, x0, W0, y0, 20), 1, 2048, 5632)
        configs["config0"]["copies"] = len(W0)
        del W0
        W2 = _weights(torch, 12288, 4096, rot_copies(12288, 4096), dev, 51)
        c2 = {}
        for m in (1, 8, 32):
            x2 = torch.randn((m, 12288), device=dev, generator=gen).half()
            y2 = torch.empty((m, 4096), device=dev, dtype=torch.float16)
            for sk in (1, 4, 8):
                c2[f"M{m}_split{sk}"] = _hbm_entry(_time_rotation(torch, ops, x2, W2, y2, 20, split_k=sk), m, 12288, 4096)
        c2["copies"] = len(W2)
        configs["config2"] = c2
        del W2
        # row-exact mode (one launch, a grid row per input row, each row the M = 1 plan) against
        # a plain GEMM of the same rows, at configs[1]'s K and two of its widths
        rx = {}
        for n in (4096, 24576):
            Wr = _weights(torch, K_DEC, n, rot_copies(K_DEC, n), dev, 53 + n)
            for m in (2, 4):
                xr = torch.randn((m, K_DEC), device=dev, generator=gen).half()
                yr = torch.empty((m, n), device=dev, dtype=torch.float16)
                e = _hbm_entry(_time_rotation(torch, ops, xr, Wr, yr, 20, fn=ops.gemm_rows_exact), m, K_DEC, n)
                e["us_plain_gemm"] = round(_time_rotation(torch, ops, xr, Wr, yr, 20), 3)
                rx[f"M{m}_N{n}"] = e
            del Wr
        configs["rows_exact"] = rx
        c3 = {}
        for n in (12288, 24576):
            W3 = _weights(torch, K_DEC, n, 3, dev, 52 + n)
            for m in (512, 2048):
                x3 = torch.randn((m, K_DEC), device=dev, generator=gen).half()
                y3 = torch.empty((m, n), device=dev, dtype=torch.float16)
                us = _time_rotation(torch, ops, x3, W3, y3, 5)
                tfl = 2.0 * m * n * K_DEC / (us * 1e-6) / 1e12
                c3[f"M{m}_N{n}"] = {"us": round(us, 1), "TFLOPs": round(tfl, 1),
                                    "mfma_frac": round(tfl / MFMA_F16_PEAK_TFLOPS, 4), "weight_copies": 3}
            del W3
        configs["config3"] = c3
        # calls between the decode batch and the prefill headline (not a configs[] shape): 33 .. 64
        # rows run as 32-row decode chunks, larger small calls cut K into ranges
        sm = {}
        Ws = _weights(torch, K_DEC, 4096, rot_copies(K_DEC, 4096), dev, 57)
        for m in (48, 128, 256):
            xs = torch.randn((m, K_DEC), device=dev, generator=gen).half()
            ys = torch.empty((m, 4096), device=dev, dtype=torch.float16)
            us = _time_rotation(torch, ops, xs, Ws, ys, 10)
            tfl = 2.0 * m * 4096 * K_DEC / (us * 1e-6) / 1e12
            sm[f"M{m}_N4096"] = {"us": round(us, 2), "TFLOPs": round(tfl, 1),
                                 "path": "decode chunks" if m <= 64 else "prefill, K ranges"}
        del Ws
        configs["small_m"] = sm

    # ---- prefill headline (configs[3], M=2048, N=24576) ----
    _progress("prefill")
    prefill = None
    if not args.no_prefill:
        M, N = 2048, 24576
        Wp = _weights(torch, K_DEC, N, 3, dev, 9)
        xp = torch.randn((M, K_DEC), device=dev, generator=gen).half()
        yp = torch.empty((M, N), device=dev, dtype=torch.float16)
        us = _time_rotation(torch, ops, xp, Wp, yp, 5)
        tflops = 2.0 * M * N * K_DEC / (us * 1e-6) / 1e12
        prefill = {"M": M, "K": K_DEC, "N": N, "us": round(us, 1), "TFLOPs": round(tflops, 1),
                   "mfma_frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4), "peak_TFLOPs": MFMA_F16_PEAK_TFLOPS,
                   # MFMA-bound: three rotated weight copies (151 MB) are enough, the launch
                   # reads 6.8x its weight bytes from L2 / the MALL either way
                   "weight_copies": 3}
        del Wp

    # ---- grouped MoE (configs[4]: E=64, top-8, H=2048, I=1024, g=128, zero points) ----
    _progress("grouped MoE")
    moe = None
    if not args.no_moe:
        moe = {T: _bench_moe(torch, ops, dev, T) for T in (16, 512)}

    # ---- fused RMSNorm + GEMM (the QKV projection after the input norm, K=4096, N=6144) ----
    _progress("RMSNorm + GEMM")
    rms = None
    if not args.no_rmsnorm:
        rms = _bench_rmsnorm(torch, ops, dev)

    line = {
        "metric": "AWQ W4A16 decode GEMV sweep throughput (algorithmic GB/s, M=1-16)",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps_timed,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic (seeded int4/zeros/scales/activations with the benchmark distributions)",
        "config": {"workload": "configs[1] decode sweep: M in {1,4,16}, K=4096, N in {4096,6144,24576}, "
                               "group 128, AutoAWQ packing", "weight_copies_rotated": copies,
                   "bytes_per_step": step_bytes},
        "roofline": roofline,
        "per_shape": per_shape,
        "configs": configs,
        "prefill": prefill,
        "moe": moe,
        "rmsnorm_fused": rms,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
