#!/usr/bin/env python3
"""Benchmark of the quantised MoE layer on one MI355X.

Workload (the metric's configuration, "MoE-layer tokens/s"): full MoE layer
forward, prefill, T=4096 tokens of fp32 N(0,1) hidden states, d_model=1024,
router [1024 -> 256] with softmax top-8, 2 shared INT8 SwiGLU experts
(ffn 2816) and 256 routed experts (ffn 256) with INT2 gate/up and INT4
down weights, fp16 group-64 scales, dropless expert sort, fp64 combine.
Weights are random (seeded), data synthetic. A step is one layer forward.

The JSON line carries, beside the contract fields:
  roofline     -- the dominant kernel's achieved rate from HIP events on the
                  forward's stream (algorithmic ops per launch / average
                  launch time) against MI355X's dense int8 MFMA peak;
  cpu_baseline -- the reference CPU kernels (oracle/_ref, built from the
                  reference sources) timed on a bounded token sample on this
                  host, or the oracle restatement when _ref is absent;
  sub          -- the other benchmark shapes: W8A8 GEMM 64x1024x1024,
                  shared-expert decode M in {1,4,16}, routed decode T=16,
                  the full decode layer at T=16, the E=512 stress
                  grouped GEMM, the batched MoE backward (training and
                  layer shapes), the GDN-2 decode step and prefill, and the
                  INT8 attention projection.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

INT8_PEAK = 5.0e15  # MI355X dense int8 MFMA, ops/s
HBM_PEAK = 8.0e12   # bytes/s


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-sub", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    p.add_argument("--cpu-sub-seconds", type=float, default=1.0,
                   help="time budget per case of the other shapes' CPU baselines")
    p.add_argument("--serial", action="store_true",
                   help="run the timed region with every stage in order on one stream "
                        "(as the profiled pass does), so that a kernel trace of the "
                        "whole run sees each kernel alone on the GPU")
    p.add_argument("--decode-only", action="store_true",
                   help="run only the full decode-layer sub-benchmark (T=16, router, "
                        "two shared and 256 routed experts) and print its JSON line; "
                        "the workload of the decode kernel-trace profile")
    p.add_argument("--only", choices=["w8a8_64", "shared_decode", "routed_decode", "stress",
                                      "bwd", "gdn2", "proj", "vendor", "dropin", "calib"],
                   help="run one of the other shapes' benchmarks alone and print its JSON "
                        "(the workloads of their kernel-trace profiles)")
    p.add_argument("--copy-probe", action="store_true",
                   help="also run a plain 256 MiB device copy (the reference kernel "
                        "for scaling HBM byte counters)")
    return p.parse_args()


def copy_probe(torch):
    """Two plain device copies of 256 MiB (the kernel of known size that
    scales the HBM byte counters FETCH_SIZE and WRITE_SIZE)."""
    src = torch.empty(64 << 20, device="cuda", dtype=torch.float32).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def make_layer(torch, api, n, h, E, k, S, hs, T, seed, router=True):
    g = torch.Generator(device="cuda").manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g, device="cuda", dtype=torch.float32)  # noqa
    W = dict(Wgate=rn(E, n) / n ** 0.5 if router else None,
             Wg=rn(E, h, n) / n ** 0.5, Wu=rn(E, h, n) / n ** 0.5, Wd=rn(E, h, n) / h ** 0.5)
    if S:
        W.update(Wg_s=rn(S, hs, n) / n ** 0.5, Wu_s=rn(S, hs, n) / n ** 0.5,
                 Wd_s=rn(S, hs, n) / hs ** 0.5)
    else:
        W.update(Wg_s=None, Wu_s=None, Wd_s=None)
    L = api.MoE(n, h, E, k, S, hs, T, W["Wgate"], W["Wg"], W["Wu"], W["Wd"], W["Wg_s"],
                W["Wu_s"], W["Wd_s"])
    return L, W


def time_fn(torch, fn, steps, warmup, stream):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return wall, e0.elapsed_time(e1) / steps


def time_graph(torch, fn, calls, reps, stream):
    """Device time per call (ms) of `calls` back-to-back calls of fn captured
    into one HIP graph: the replay launches every kernel with no host work
    between them, so a call that is shorter than its host-side enqueue
    (ctypes, argument checks, the launch API) is timed by its kernels and the
    gaps between them alone. fn must only launch kernels (no allocation, no
    synchronisation); median over reps replays."""
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for _ in range(calls):
            fn()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        g.replay()  # warm
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            g.replay()
            e1.record(stream)
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) / calls)
    del g
    return sorted(ts)[len(ts) // 2]


def spread_fn(torch, fn, n, stream):
    """Median and median absolute deviation (ms) of n single-step times, from
    an event recorded after every step (the reference's methodology,
    bench/common/bench_common.h:39-45). Run outside the timed region: each
    event adds its marker to the step it closes."""
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    torch.cuda.synchronize()
    evs[0].record(stream)
    for i in range(1, n + 1):
        fn()
        evs[i].record(stream)
    torch.cuda.synchronize()
    per = sorted(evs[i - 1].elapsed_time(evs[i]) for i in range(1, n + 1))
    med = per[n // 2]
    mad = sorted(abs(x - med) for x in per)[n // 2]
    return med, mad


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: there is no multi-GPU path "
              "(tokens and experts would shard across GPUs, not built here); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import jimotono_amd.api as api

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    assert api.lib().jt_hip_init(0) == 0
    # a dedicated stream for the layer and its timing events
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    if args.decode_only or args.only:
        if args.copy_probe:
            copy_probe(torch)
        res = ({"decode_layer_T16": decode_layer(torch, api, stream, args.steps, args.warmup)}
               if args.decode_only else sub_benchmarks(np, torch, api, stream, only=args.only))
        print(json.dumps(res), flush=True)
        return

    # ---------------- main workload: full layer prefill ----------------
    n, h, E, k, S, hs, T = 1024, 256, 256, 8, 2, 2816, 4096
    L, W = make_layer(torch, api, n, h, E, k, S, hs, T, seed=1234)
    g = torch.Generator(device="cuda").manual_seed(99)
    X = torch.randn(T, n, generator=g, device="cuda", dtype=torch.float32)
    Y = torch.empty(T, n, device="cuda", dtype=torch.float32)

    def step():
        rc = L.fwd(X, Y, stream)
        if rc != 0:
            raise RuntimeError(f"jt_hip_moe_fwd rc={rc}")

    # Untimed diagnostic passes first, then the W warmup steps and the K timed
    # steps back to back. After an idle stretch the GPU runs the first ~10
    # steps 10-25% slower (measured 360-420 us, then about 330 us per step)
    # while its clocks come back; the passes keep that ramp out of the timed
    # steps, so `value` is the layer's steady-state rate.
    step()  # first call: kernel attributes and workspaces
    torch.cuda.synchronize()
    # single-step spread (its median is robust to the ramp); with --serial
    # every pass runs its stages in stream order, as the timed region does
    L.set_profiling(args.serial)
    step_med, step_mad = spread_fn(torch, step, max(args.steps, 50), stream)
    L.set_profiling(False)
    assert api.sync_errors(stream) == 0
    # profiled pass: every stage in order on the stream, HIP events around
    # each stage give per-kernel launch durations for the roofline
    L.set_profiling(True)
    L.stage_times()  # reset
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    stages, count = L.stage_times()
    L.set_profiling(False)
    assert api.sync_errors(stream) == 0
    serial_ms = sum(stages.values()) / count

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    assert api.sync_errors(stream) == 0
    if args.copy_probe:
        copy_probe(torch)
    # timed region: the production path (shared experts overlap the routed
    # path on side streams), or with --serial every stage in stream order
    if args.serial:
        L.set_profiling(True)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ev_ms = e0.elapsed_time(e1) / args.steps
    L.set_profiling(False)
    assert api.sync_errors(stream) == 0
    ms_per_step = wall_ms
    tokens_per_s = T / (ms_per_step / 1e3)


    # algorithmic work per stage launch
    ops = {
        "shared_gateup": 2.0 * T * (2 * hs) * n,   # per shared expert
        "shared_down": 2.0 * T * n * hs,
        "routed_gateup": 2.0 * T * k * (2 * h) * n,
        "routed_down": 2.0 * T * k * n * h,
    }
    # the library runs the S shared gate/ups as one GEMM (gate/up panels
    # concatenated along N) when S >= 2, T > 64 and 2 * hs fills whole
    # 128-channel panels with S * 2 * hs a multiple of 256
    fused = S >= 2 and T > 64 and (2 * hs) % 128 == 0 and (S * 2 * hs) % 256 == 0
    launches = {"shared_gateup": 1 if fused else S, "shared_down": S, "routed_gateup": 1,
                "routed_down": 1}
    per_expert = {"shared_gateup": S, "shared_down": S, "routed_gateup": 1, "routed_down": 1}
    ops = {st: v * per_expert[st] / launches[st] for st, v in ops.items()}  # per launch
    per_launch = {s: stages[s] / (count * launches.get(s, 1)) for s in stages}
    dom = max(ops, key=lambda s: stages[s])
    dom_ms = per_launch[dom]
    achieved = ops[dom] / (dom_ms / 1e3)
    total_ops = 2.0 * T * (S * (2 * hs * n + n * hs) + k * (2 * h * n + n * h))
    traffic = measured_traffic(dom)
    roofline = {"bound": "mfma", "kernel": dom, "achieved": achieved / 1e12,
                "peak": INT8_PEAK / 1e12, "unit": "TFLOP/s",
                "frac": achieved / INT8_PEAK,
                "traffic": None if traffic is None else traffic["bytes"],
                "ops_per_launch": ops[dom], "avg_launch_ms": dom_ms}
    if traffic is not None:
        roofline["traffic_source"] = traffic["source"]

    out = {
        "metric": "MoE-layer tokens/s; int8 TOPS (prefill) and HBM GB/s (decode) vs roofline",
        "value": tokens_per_s, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_per_step, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,1) activations, random-init weights)",
        "serial": bool(args.serial),
        "config": {"workload": "moe_layer_prefill", "tokens": T, "d_model": n,
                   "routed_experts": E, "expert_ffn": h, "topk": k, "shared_experts": S,
                   "shared_ffn": hs, "routed_quant": "INT2 gate/up, INT4 down, fp16 g64",
                   "shared_quant": "W8A8 per-channel",
                   "router": "exact fp64 top-8 (int8 MFMA bounds, fp64 candidates)",
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "layer_int8_tops": total_ops / (ms_per_step / 1e3) / 1e12,
        "layer_mfma_frac": total_ops / (ms_per_step / 1e3) / INT8_PEAK,
        "event_ms_per_step": ev_ms,
        "serialized_ms_per_step": serial_ms,
        "stages_ms_per_step": {s: v / count for s, v in stages.items()},
        "step_ms_median": step_med, "step_ms_mad": step_mad,
        "step_spread_samples": max(args.steps, 50),
        "untimed_before_warmup": f"1 step, {max(args.steps, 50)} single-step timings, "
                                 f"{args.steps} profiled steps",
    }

    # ---------------- PCIe-inclusive rate (never the value) ----------------
    # the same forward when the caller hands over host buffers: pinned X in,
    # the layer, pinned Y out, in stream order on the one stream
    Xh = torch.empty(T, n, dtype=torch.float32, pin_memory=True)
    Xh.copy_(X.cpu())
    Yh = torch.empty(T, n, dtype=torch.float32, pin_memory=True)

    def host_step():
        X.copy_(Xh, non_blocking=True)
        step()
        Yh.copy_(Y, non_blocking=True)

    if args.serial:  # keep every kernel alone on the GPU for a kernel trace
        L.set_profiling(True)
    _, pcie_ms = time_fn(torch, host_step, max(2, args.steps // 2), 2, stream)
    L.set_profiling(False)
    assert api.sync_errors(stream) == 0
    out["pcie_inclusive"] = {"tokens_per_s": T / (pcie_ms / 1e3), "ms_per_step": pcie_ms,
                             "bytes_over_pcie_per_step": 2 * T * n * 4}
    del Xh, Yh

    # ---------------- CPU baseline ----------------
    if not args.no_cpu_baseline:
        try:
            out["cpu_baseline"] = cpu_baseline(np, torch, W, X, n, h, E, k, S, hs,
                                               args.cpu_seconds)
        except Exception as ex:  # reported, never fatal
            out["cpu_baseline"] = {"error": repr(ex)}
    del L
    torch.cuda.empty_cache()

    if not args.no_sub:
        out["sub"] = sub_benchmarks(np, torch, api, stream)
        if not args.no_cpu_baseline:
            # the reference CPU path of the other shapes, one pinned core
            try:
                from oracle.cpu_bench import decode_and_stress
                cb = decode_and_stress(args.cpu_sub_seconds)
                host = {k: cb.get(k) for k in ("host_cpu", "cores", "core", "kind", "vnni")
                        if k in cb}
                for build, res in cb.items():
                    if not isinstance(res, dict):
                        continue
                    for shape, r in res.items():
                        tgt = "stress_prefill_E512" if shape.startswith("stress") else shape
                        if tgt in out["sub"]:
                            out["sub"][tgt].setdefault("cpu_baseline", dict(host))[build] = r
            except Exception as ex:  # reported, never fatal
                out["sub_cpu_baseline_error"] = repr(ex)
    print(json.dumps(out), flush=True)


def measured_traffic(stage):
    """HBM bytes per launch of a stage's kernel from the committed rocprofv3
    PMC summary (FETCH_SIZE and WRITE_SIZE, each scaled by the same counter's
    reading for a plain copy of known size), or None when none is recorded."""
    path = os.path.join(ROOT, "profiles", f"{stage}_pmc_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return {"bytes": float(line.split(":", 1)[1]),
                    "source": os.path.relpath(path, ROOT)}
    return None


def cpu_baseline(np, torch, W, X, n, h, E, k, S, hs, seconds):
    """Reference CPU path on a bounded token sample, single core.

    Routed experts: jt_lowbit_gemm_lut (gate/up bits 2, down bits 4) per
    touched expert on the dropless permutation of the sample; shared experts:
    jt_w8a8_quant_per_channel of the token rows then jt_w8a8_gemm_per_channel
    row by row (one activation scale per call); routing: the reference's
    jt_routing_topk on the layer's own logits. Sample grows until `seconds`.
    """
    from oracle.pyoracle import RefLib, ref_available
    Xh = X[:256].cpu().numpy()
    Wg = W["Wg"].cpu().numpy()
    Wu = W["Wu"].cpu().numpy()
    Wd = W["Wd"].cpu().numpy()
    Wgate = W["Wgate"].cpu().numpy()
    Wgs, Wus, Wds = (W[x].cpu().numpy() for x in ("Wg_s", "Wu_s", "Wd_s"))
    if not ref_available():
        return cpu_baseline_port(np, Xh, Wgate, Wg, Wu, Wd, Wgs, Wus, Wds, n, h, E, k, S, hs,
                                 seconds)
    R = RefLib()
    # weights pre-transposed the way the reference driver hands them to
    # jt_lowbit_gemm_lut (src/moe_layer.c:1302-1331): gate/up [n][h]
    WgT = np.ascontiguousarray(np.transpose(Wg, (0, 2, 1)))
    WuT = np.ascontiguousarray(np.transpose(Wu, (0, 2, 1)))
    # shared experts: weights quantised once per output channel, laid out as
    # the reference's B[K][N] (src/moe_layer.c:164-274 quantises per call;
    # that cost is left out here in the CPU's favour)
    shared = []
    for sidx in range(S):
        _, qg, sg = R.quant_rows(np.ascontiguousarray(Wgs[sidx]))
        _, qu, su = R.quant_rows(np.ascontiguousarray(Wus[sidx]))
        _, qd, sdn = R.quant_rows(np.ascontiguousarray(Wds[sidx].T))
        shared.append((np.ascontiguousarray(qg.T), sg, np.ascontiguousarray(qu.T), su,
                       np.ascontiguousarray(qd.T), sdn))

    def run(tok):
        Xs = Xh[:tok]
        logits = (Xs.astype(np.float64) @ Wgate.T.astype(np.float64)).astype(np.float32)
        ids = np.zeros((tok, k), np.int64)
        for t in range(tok):
            _, ids[t], _ = R.topk(logits[t], k)
        for e in np.unique(ids):
            rows = np.nonzero((ids == e).any(axis=1))[0]
            Xe = np.ascontiguousarray(Xs[rows])
            _, G = R.lowbit_gemm_lut(Xe, WgT[e], 2)
            _, U = R.lowbit_gemm_lut(Xe, WuT[e], 2)
            Sg = (G / (1 + np.exp(-G.astype(np.float64))) * U).astype(np.float32)
            R.lowbit_gemm_lut(Sg, Wd[e], 4)
        _, Xq, sx = R.quant_rows(Xs)
        for Bg, sg, Bu, su, Bd, sdn in shared:
            Ss = np.zeros((tok, hs), np.float32)
            for t in range(tok):
                _, G = R.gemm_per_channel(Xq[t:t + 1], Bg, sx[t], sg)
                _, U = R.gemm_per_channel(Xq[t:t + 1], Bu, sx[t], su)
                Ss[t] = (G / (1 + np.exp(-G.astype(np.float64))) * U)[0]
            _, Sq, ss = R.quant_rows(Ss)
            for t in range(tok):
                R.gemm_per_channel(Sq[t:t + 1], Bd, ss[t], sdn)

    from oracle.cpu_bench import host_info, pinned
    tok, el = 2, 0.0
    with pinned() as pn:
        while True:
            t0 = time.perf_counter()
            run(tok)
            el = time.perf_counter() - t0
            if el >= seconds or tok >= 256:
                break
            tok = min(256, max(tok * 2, int(tok * seconds / max(el, 1e-3) * 0.9)))
    return {"value": tok / el, "unit": "tokens/s", "cores": 1, "kind": "reference",
            "host_cpu": host_info()[0], "core": pn.core,
            "sample": f"{tok} tokens of the same layer (routed: reference "
                      "jt_lowbit_gemm_lut T-MAC per touched expert; shared: reference "
                      "W8A8 quant + gemm_per_channel per token row; top-k: reference "
                      f"jt_routing_topk), {el:.1f} s on one pinned core, default "
                      "reference build (-mavx2)",
            "seconds": el}


def cpu_baseline_port(np, Xh, Wgate, Wg, Wu, Wd, Wgs, Wus, Wds, n, h, E, k, S, hs, seconds):
    from oracle.pyoracle import Oracle
    O = Oracle()
    OL = O.moe_q(n, h, E, k, S, hs, Wgate, Wg, Wu, Wd, Wgs, Wus, Wds)
    tok, el = 2, 0.0
    while True:
        t0 = time.perf_counter()
        OL.fwd(Xh[:tok])
        el = time.perf_counter() - t0
        if el >= seconds or tok >= 256:
            break
        tok = min(256, max(tok * 2, int(tok * seconds / max(el, 1e-3) * 0.9)))
    return {"value": tok / el, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"{tok} tokens of the same layer through the oracle's C "
                      f"restatement, {el:.1f} s single-threaded", "seconds": el}


def decode_layer(torch, api, stream, steps, warmup):
    """Full decode layer: T=16 tokens through the router (top-8 of 256), two
    shared experts (ffn 2816) and the routed experts (ffn 256), d=1024. Four
    layer copies (90 MB of weights each) rotate so the weights stream from
    HBM, as they would through a model's layers."""
    n, h, E, k, S, hs, T = 1024, 256, 256, 8, 2, 2816, 16
    layers = [make_layer(torch, api, n, h, E, k, S, hs, T, seed=900 + c)[0] for c in range(4)]
    X = torch.randn(T, n, device="cuda")
    Y = torch.empty(T, n, device="cuda")
    it = [0]

    def step():
        rc = layers[it[0] % len(layers)].fwd(X, Y, stream)
        assert rc == 0
        it[0] += 1
    # the spread pass first: it also brings the clocks up before the timing
    med, mad = spread_fn(torch, step, 64, stream)
    _, ev = time_fn(torch, step, max(steps, 8) * 4, max(warmup, 2) * 4, stream)
    gr = time_graph(torch, step, 16, 5, stream)  # four passes over the 4 copies
    assert api.sync_errors(stream) == 0
    # weight bytes one forward reads: the shared experts, the fp32 gate and
    # the routed experts its tokens touch (counted on layer 0's routing)
    import numpy as np
    assert layers[0].fwd(X, Y, stream) == 0
    torch.cuda.synchronize()
    touched = len(np.unique(layers[0].read(api.BUF_IDS, np.int32, (T, k))))
    per_expert = 2 * h * n // 4 + n * h // 2 + 2 * (2 * h * n // 64 + n * h // 64)
    wbytes = S * (3 * hs * n + 4 * (2 * hs + n)) + 4 * E * n + touched * per_expert
    del layers
    torch.cuda.empty_cache()
    return {"us_per_layer": ev * 1e3, "us_median": med * 1e3, "us_mad": mad * 1e3,
            "tokens": T, "touched_experts": touched,
            "weight_bytes": wbytes, "gbps": wbytes / (ev / 1e3) / 1e9,
            "hbm_frac": wbytes / (ev / 1e3) / HBM_PEAK,
            "graph_us_per_layer": gr * 1e3, "graph_hbm_frac": wbytes / (gr / 1e3) / HBM_PEAK}


def sub_benchmarks(np, torch, api, stream, only=None):
    res = {}
    want = lambda name: only is None or only == name  # noqa: E731
    if want("w8a8_64"):
        res.update(w8a8_64_bench(np, torch, api, stream))
    if want("shared_decode"):
        res.update(shared_decode_bench(np, torch, api, stream))
    if want("routed_decode"):
        res.update(routed_decode_bench(np, torch, api, stream))
    if only is None:
        res["decode_layer_T16"] = decode_layer(torch, api, stream, 10, 2)
    if want("stress"):
        res.update(stress_bench(np, torch, api, stream))
    if want("bwd"):
        for name, shape in BWD_SHAPES.items():
            res[name] = bwd_bench(np, torch, api, stream, *shape)
    if want("gdn2"):
        res.update(gdn2_bench(np, torch, api, stream))
    if want("proj"):
        res.update(proj_bench(np, torch, api, stream))
    if want("vendor"):
        res.update(vendor_bench(np, torch, api, stream))
    if want("dropin"):
        res.update(dropin_bench(np, torch, api))
    if want("calib"):
        res["calibration"] = calib_bench()
    return res


def calib_bench(blocks=512, iters=4000):
    """Issue rates of this GPU from libjimotono_calib.so (calib/calib.hip):
    the int8 MFMA rate alone, the fp32 and fp64 FMA rates alone, and how
    much of the shorter of the two the GPU hides when MFMAs and FMAs come
    from different waves of one SIMD (split) or from the same wave (same):
    overlap = (t_mfma + t_valu - t_mixed) / min(t_mfma, t_valu), 1 for
    perfect overlap and 0 when the two run one after the other. Then the
    MFMA rate with LDS-fed operands (and a barrier per 16 MFMAs), and the
    128x256 tile GEMM's rate with its operands in HBM or aliased into L2.
    512 blocks of 8 waves: 4 waves per SIMD. Times per wave iteration are in
    ns per SIMD (each SIMD runs blocks * 8 / 1024 waves)."""
    import ctypes as C
    Lc = C.CDLL(os.path.join(ROOT, "jimotono_amd", "libjimotono_calib.so"))
    Lc.jt_calib_issue.argtypes = [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_float)]
    Lc.jt_calib_tile.argtypes = [C.c_int, C.POINTER(C.c_float), C.POINTER(C.c_double)]
    t = []
    for mode in range(9):
        ms = C.c_float()
        rc = Lc.jt_calib_issue(mode, blocks, iters, C.byref(ms))
        assert rc == 0, f"jt_calib_issue({mode}) rc={rc}"
        t.append(ms.value)
    per_simd = iters * blocks * 8 / 1024  # wave iterations per SIMD
    ns = lambda m: t[m] * 1e6 / per_simd  # noqa: E731
    mfma_ops = blocks * 8 * iters * 16 * 32768.0
    tops = lambda m, frac=1.0: mfma_ops * frac / (t[m] * 1e-3) / 1e12  # noqa: E731
    ovl = lambda a, b, mix: (a + b - mix) / min(a, b)  # noqa: E731
    res = {
        "blocks": blocks, "iters": iters, "waves_per_simd": blocks * 8 // 1024,
        "mfma_i8_16x16x64_tops": tops(0),
        "mfma_i8_ns_each": ns(0) / 16,
        "fp32_fma_wave64_ns_each": ns(1) / 64,
        "fp64_fma_wave64_ns_each": ns(4) / 64,
        "overlap_fp32_split_waves": ovl(t[0] / 2, t[1] / 2, t[2]),
        "overlap_fp32_same_wave": ovl(t[0], t[1], t[3]),
        "overlap_fp64_split_waves": ovl(t[0] / 2, t[4] / 2, t[5]),
        "overlap_fp64_same_wave": ovl(t[0], t[4], t[6]),
        "mfma_lds_fed_tops": tops(7),
        "mfma_lds_fed_barrier_tops": tops(8),
        "ms": dict(zip(["mfma", "fp32", "mfma_fp32_split", "mfma_fp32_same", "fp64",
                        "mfma_fp64_split", "mfma_fp64_same", "mfma_lds", "mfma_lds_barrier"],
                       t)),
    }
    tile = {}
    for which, name in enumerate(["hbm_A_W_C", "C_aliased", "A_C_aliased", "all_in_L2"]):
        us, tp = C.c_float(), C.c_double()
        rc = Lc.jt_calib_tile(which, C.byref(us), C.byref(tp))
        assert rc == 0, f"jt_calib_tile({which}) rc={rc}"
        tile[name] = {"us": us.value, "tops": tp.value}
    res["tile_128x256_k1024_plain"] = tile
    return res


DROPIN_MODES = {"fp32": (0, 0), "w8a8": (1, 0), "lowbit_fakequant": (0, 1),
                "lowbit_lut": (0, 2), "w8a8_and_lowbit_fakequant": (1, 1)}


def dropin_bench(np, torch, api):
    """The drop-in jt_moe_fwd_batch (host pointers, the reference's own
    layer entry) at the reference trainer's shape: T=512 tokens (seq 128 x
    batch 4), d=64, h=32, E=8, top-2, one shared expert, cap 1.5
    (bench/kernel/train_tinystories.c:78-81, 1141-1144), in each of the
    process-flag modes. Every call copies X and the fp32 weights over PCIe,
    runs the forward and copies Y, ids, weights and the sort back, as the
    reference's callers expect; the time per call is wall clock (median of
    the calls after two warm-up calls)."""
    T, n, h, E, k, S = 512, 64, 32, 8, 2, 1
    rng = np.random.default_rng(512)
    X = rng.standard_normal((T, n)).astype(np.float32)
    W = [(rng.standard_normal(sh) / np.sqrt(sh[-1])).astype(np.float32)
         for sh in [(E, n), (E, h, n), (E, h, n), (E, h, n), (S, h, n), (S, h, n), (S, h, n)]]
    lib = api.lib()
    res = {}
    for name, (w8, lb) in DROPIN_MODES.items():
        assert lib.jt_w8a8_set_enabled(w8) == 0 and lib.jt_lowbit_set_mode(lb) == 0
        try:
            for _ in range(2):
                assert api.moe_fwd_batch(X, *W, k, 1.5)["rc"] == 0
            ts = []
            for _ in range(30):
                t0 = time.perf_counter()
                r = api.moe_fwd_batch(X, *W, k, 1.5)
                ts.append(time.perf_counter() - t0)
                assert r["rc"] == 0
        finally:
            lib.jt_w8a8_set_enabled(0)
            lib.jt_lowbit_set_mode(0)
        med = float(np.median(ts))
        res[name] = {"ms_per_call": med * 1e3, "tokens_per_s": T / med,
                     "mad_ms": float(np.median(np.abs(np.array(ts) - med))) * 1e3}
    # the trainer's backward through the drop-in jt_moe_bwd_batch (flags off:
    # the forward's caches and sort, a random upstream gradient)
    f = api.moe_fwd_batch(X, *W, k, 1.5, caches=True)
    assert f["rc"] == 0
    dY = rng.standard_normal((T, n)).astype(np.float32)
    bargs = [dY, X, *W, f["ids"], f["w"], f["Gsel"], f["Usel"], f["Ysel"], f["Gs"], f["Us"],
             f["perm"], f["off"], f["drop"], k]
    for _ in range(2):
        assert api.moe_bwd_batch(*bargs)["rc"] == 0
    ts = []
    for _ in range(30):
        t0 = time.perf_counter()
        assert api.moe_bwd_batch(*bargs)["rc"] == 0
        ts.append(time.perf_counter() - t0)
    bmed = float(np.median(ts))
    pcie = 4 * (T * n + E * n + 3 * E * h * n + 3 * S * h * n) + 4 * T * n + 12 * T * k
    return {"dropin_moe_fwd_batch_T512_train": {
        "shape": {"tokens": T, "d_model": n, "expert_ffn": h, "experts": E, "topk": k,
                  "shared": S, "cap_factor": 1.5},
        "includes_pcie": True, "host_bytes_each_way_per_call": pcie, "modes": res,
        "bwd_ms_per_call": bmed * 1e3,
        "bwd_mad_ms": float(np.median(np.abs(np.array(ts) - bmed))) * 1e3}}


def vendor_bench(np, torch, api, stream):
    """The shared experts' two prefill GEMM shapes through this library's
    W8A8 GEMM (int8 MFMA, fp32 output with the per-row x per-channel scale
    epilogue) and through torch._int_mm (the vendor int8 GEMM library, int32
    output, no epilogue), same int8 operands, timed alike: a reference point
    for the int8 main loop on these shapes."""
    res = {}
    for M, N, K in ((4096, 5632, 1024), (4096, 1024, 2816)):
        g = torch.Generator(device="cuda").manual_seed(N + K)
        A = torch.randint(-127, 128, (M, K), generator=g, device="cuda", dtype=torch.int8)
        Bkn = torch.randint(-127, 128, (K, N), generator=g, device="cuda", dtype=torch.int8)
        sA = torch.rand(M, generator=g, device="cuda") * 9e-3 + 1e-3
        sB = torch.rand(N, generator=g, device="cuda") * 9e-3 + 1e-3
        Wq = api.W8A8(Bq_kn=Bkn, sB=sB)
        C = torch.empty(M, N, device="cuda")
        _, ours = time_fn(torch, lambda: Wq.gemm(A, sA, C, stream), 50, 5, stream)
        Bt = Bkn.t().contiguous().t()  # column-major B, the library's preferred layout
        _, ven = time_fn(torch, lambda: torch._int_mm(A, Bt), 50, 5, stream)
        ops = 2.0 * M * N * K
        res[f"int8_gemm_{M}x{N}x{K}"] = {
            "ours_us": ours * 1e3, "ours_tops": ops / (ours / 1e3) / 1e12,
            "vendor_int_mm_us": ven * 1e3, "vendor_tops": ops / (ven / 1e3) / 1e12,
            "ours_over_vendor_time": ours / ven}
        del Wq, A, Bkn, Bt, C
    torch.cuda.empty_cache()
    return res


def w8a8_64_bench(np, torch, api, stream):
    """W8A8 GEMM 64x1024x1024 with per-row activation scales."""
    res = {}
    M, N, K = 64, 1024, 1024
    g = torch.Generator(device="cuda").manual_seed(5)
    Bq = torch.randint(-127, 128, (K, N), generator=g, device="cuda", dtype=torch.int8)
    sB = torch.rand(N, generator=g, device="cuda") * 9e-3 + 1e-3
    Wq = api.W8A8(Bq_kn=Bq, sB=sB)
    Aq = torch.randint(-127, 128, (M, K), generator=g, device="cuda", dtype=torch.int8)
    sA = torch.rand(M, generator=g, device="cuda") * 9e-3 + 1e-3
    Cc = torch.empty(M, N, device="cuda")
    wall, ev = time_fn(torch, lambda: Wq.gemm(Aq, sA, Cc, stream), 200, 20, stream)
    gr = time_graph(torch, lambda: Wq.gemm(Aq, sA, Cc, stream), 200, 5, stream)
    nbytes = M * K + N * K + 4 * (M + N) + 4 * M * N
    res["w8a8_gemm_64x1024x1024"] = {"us_per_call": ev * 1e3,
                                     "host_us_per_call": wall * 1e3,
                                     "tops": 2 * M * N * K / (ev / 1e3) / 1e12,
                                     "mfma_frac": 2 * M * N * K / (ev / 1e3) / INT8_PEAK,
                                     "bytes": nbytes,
                                     "gbps": nbytes / (ev / 1e3) / 1e9,
                                     "hbm_frac": nbytes / (ev / 1e3) / HBM_PEAK,
                                     "peak_gbps": HBM_PEAK / 1e9,
                                     "graph_us_per_call": gr * 1e3,
                                     "graph_hbm_frac": nbytes / (gr / 1e3) / HBM_PEAK}
    del Wq
    return res


def shared_decode_bench(np, torch, api, stream):
    """Shared-expert decode, M in {1,4,16}; 40 rotating weight copies
    (> 256 MB MALL) so every call streams its weights from HBM."""
    res = {}
    n, hs = 1024, 2816
    copies = 40
    Fs = []
    for c in range(copies):
        gw = torch.Generator(device="cuda").manual_seed(100 + c)
        Fs.append(api.FFN(torch.randn(hs, n, generator=gw, device="cuda") / 32,
                          torch.randn(hs, n, generator=gw, device="cuda") / 32,
                          torch.randn(hs, n, generator=gw, device="cuda") / 53))
    wbytes = 3 * hs * n + 4 * (2 * hs + n)
    for m in (1, 4, 16):
        Xd = torch.randn(m, n, device="cuda")
        Yd = torch.empty(m, n, device="cuda")
        it = [0]

        def fstep():
            Fs[it[0] % copies].fwd(Xd, Yd, stream)
            it[0] += 1
        _, ev = time_fn(torch, fstep, 4 * copies, copies, stream)
        gr = time_graph(torch, fstep, copies, 5, stream)  # one call per copy
        res[f"shared_decode_M{m}"] = {"us_per_expert": ev * 1e3,
                                      "gbps": (wbytes + 8 * m * n) / (ev / 1e3) / 1e9,
                                      "hbm_frac": (wbytes + 8 * m * n) / (ev / 1e3) / HBM_PEAK,
                                      "peak_gbps": HBM_PEAK / 1e9,
                                      "graph_us_per_expert": gr * 1e3,
                                      "graph_hbm_frac": (wbytes + 8 * m * n) / (gr / 1e3)
                                      / HBM_PEAK}
    del Fs
    torch.cuda.empty_cache()
    return res


def routed_decode_bench(np, torch, api, stream):
    """Routed decode: T=16, E=256, d=1024, f=256, k=8, Zipf(1.1) ids given."""
    res = {}
    n, h, E, k, T = 1024, 256, 256, 8, 16
    rng = np.random.default_rng(16)
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    ids = np.stack([rng.choice(E, k, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    w = rng.uniform(0, 1, (T, k)).astype(np.float32)
    w /= w.sum(1, keepdims=True)
    touched = len(np.unique(ids))
    layers = []
    for c in range(8):  # 8 layers x 73 MB of routed weights rotate past the MALL
        Lr, _ = make_layer(torch, api, n, h, E, k, 0, 0, T, seed=500 + c, router=False)
        layers.append(Lr)
    dids = torch.from_numpy(ids).cuda()
    dw = torch.from_numpy(w).cuda()
    Xr = torch.randn(T, n, device="cuda")
    Yr = torch.empty(T, n, device="cuda")
    it = [0]

    def rstep():
        rc = layers[it[0] % len(layers)].fwd_routed(Xr, dids, dw, Yr, stream)
        assert rc == 0
        it[0] += 1
    _, ev = time_fn(torch, rstep, 40, 8, stream)
    gr = time_graph(torch, rstep, 40, 5, stream)  # five passes over the 8 layers
    rbytes = touched * (2 * h * n // 4 + n * h // 2 + 2 * (2 * h * n // 64 + n * h // 64))
    res["routed_decode_T16"] = {"us_per_layer": ev * 1e3, "touched_experts": touched,
                                "weight_bytes": rbytes,
                                "gbps": rbytes / (ev / 1e3) / 1e9,
                                "hbm_frac": rbytes / (ev / 1e3) / HBM_PEAK,
                                "peak_gbps": HBM_PEAK / 1e9,
                                "graph_us_per_layer": gr * 1e3,
                                "graph_hbm_frac": rbytes / (gr / 1e3) / HBM_PEAK}
    del layers
    torch.cuda.empty_cache()
    return res


def stress_bench(np, torch, api, stream):
    """Stress prefill: T=16384, d=2048, E=512, f=512, k=8, Zipf(1.1) ids."""
    res = {}
    rng = np.random.default_rng(1616)
    n, h, E, k, T = 2048, 512, 512, 8, 16384
    ids = np.stack([rng.choice(E, k, replace=False, p=(1.0 / np.arange(1, E + 1) ** 1.1)
                               / (1.0 / np.arange(1, E + 1) ** 1.1).sum())
                    for _ in range(T)]).astype(np.int32)
    w = rng.uniform(0, 1, (T, k)).astype(np.float32)
    w /= w.sum(1, keepdims=True)
    Ls, _ = make_layer(torch, api, n, h, E, k, 0, 0, T, seed=777, router=False)
    dids = torch.from_numpy(ids).cuda()
    dw = torch.from_numpy(w).cuda()
    Xs = torch.randn(T, n, device="cuda")
    Ys = torch.empty(T, n, device="cuda")
    Ls.set_profiling(True)
    Ls.stage_times()
    _, ev = time_fn(torch, lambda: Ls.fwd_routed(Xs, dids, dw, Ys, stream), 5, 2, stream)
    st, cnt = Ls.stage_times()
    Ls.set_profiling(False)
    gops = 2.0 * T * k * (2 * h * n + n * h)
    gemm_ms = (st["routed_gateup"] + st["routed_down"]) / cnt
    # Bounds of the grouped GEMM: global max(ops / peak, bytes / HBM) with the
    # weights of every expert, X int8 and Y fp32 once; and the per-expert
    # attainable time sum_e max(ops_e / peak, bytes_e / HBM), bytes_e = its
    # INT2 gate/up, INT4 down and fp16 group scales plus its gathered rows
    # (int8 in, fp32 out), as if the experts ran one after another
    wbytes = 2 * h * n // 4 + n * h // 2 + 2 * (2 * h * n // 64 + n * h // 64)
    rows = np.bincount(ids.ravel(), minlength=E).astype(np.float64)
    tot_bytes = E * wbytes + T * n + T * n * 4
    glob_ms = max(gops / INT8_PEAK, tot_bytes / HBM_PEAK) * 1e3
    ops_e = 2.0 * rows * 3 * h * n
    bytes_e = np.where(rows > 0, wbytes, 0) + rows * n * 5
    per_e_ms = float(np.maximum(ops_e / INT8_PEAK, bytes_e / HBM_PEAK).sum() * 1e3)
    res["stress_prefill_E512"] = {"ms_per_layer": ev, "grouped_gemm_ms": gemm_ms,
                                  "grouped_gemm_tops": gops / (gemm_ms / 1e3) / 1e12,
                                  "mfma_frac": gops / (gemm_ms / 1e3) / INT8_PEAK,
                                  "bound_global_ms": glob_ms,
                                  "bound_per_expert_ms": per_e_ms,
                                  "expert_bytes": wbytes, "head_expert_rows": int(rows.max()),
                                  "stages_ms": {s: v / cnt for s, v in st.items()}}
    del Ls
    torch.cuda.empty_cache()
    return res


def gdn2_bench(np, torch, api, stream):
    """GDN-2 decode: one token for 64 sequences x 8 heads of 128x128 states
    (the 1B configuration's d_model 1024 in 8 heads); each step reads and
    writes every state once. Prefill: T=4096 tokens of 8 heads in chunks of
    32. States stay in HBM."""
    res = {}
    H, dk, dv = 512, 128, 128
    g = torch.Generator(device="cuda").manual_seed(41)
    rn = lambda *s: torch.randn(*s, generator=g, device="cuda")  # noqa: E731
    S = rn(H, dk, dv) * 0.3
    q, k, b = rn(H, dk), rn(H, dk), torch.rand(H, dk, generator=g, device="cuda")
    a = torch.rand(H, dk, generator=g, device="cuda") * 0.1 + 0.9
    v, w = rn(H, dv), torch.rand(H, dv, generator=g, device="cuda")
    O = torch.empty(H, dv, device="cuda")
    _, ev = time_fn(torch, lambda: api.gdn2_decode_device(S, O, q, k, v, b, w, a, stream), 50,
                    5, stream)
    assert api.sync_errors(stream) == 0
    nbytes = H * (2 * dk * dv * 4 + 4 * dk * 4 + 3 * dv * 4)
    res["gdn2_decode_H512"] = {"us_per_step": ev * 1e3, "heads": H, "dk": dk, "dv": dv,
                               "state_bytes_rw": nbytes, "gbps": nbytes / (ev / 1e3) / 1e9,
                               "hbm_frac": nbytes / (ev / 1e3) / HBM_PEAK}
    del S, O
    H, T, C = 8, 4096, 32
    S = rn(H, dk, dv) * 0.3
    Q, K, B = rn(H, T, dk), rn(H, T, dk), torch.rand(H, T, dk, generator=g, device="cuda")
    A = torch.rand(H, T, dk, generator=g, device="cuda") * 0.1 + 0.9
    V, W = rn(H, T, dv), torch.rand(H, T, dv, generator=g, device="cuda")
    Out = torch.empty(H, T, dv, device="cuda")
    ws = [None]

    def pstep():
        rc, ws[0] = api.gdn2_prefill_device(S, Out, Q, K, V, B, W, A, C, ws=ws[0], stream=stream)
        assert rc == 0
    _, ev = time_fn(torch, pstep, 3, 1, stream)
    assert api.sync_errors(stream) == 0
    # fp32 work of the WY form per chunk and head (multiplies and adds):
    # B, Out and the state update 3 x 2 C dk dv, the solve and P terms C^2 dv
    flops = H * (T // C) * (6.0 * C * dk * dv + 2.0 * C * C * dv)
    res["gdn2_prefill_T4096_H8"] = {"ms": ev, "tokens_per_s": H * T / (ev / 1e3),
                                    "heads": H, "T": T, "chunk": C, "dk": dk, "dv": dv,
                                    "gflops": flops / (ev / 1e3) / 1e9}
    del S, Q, K, B, A, V, W, Out, ws
    torch.cuda.empty_cache()
    return res


def proj_bench(np, torch, api, stream):
    """The INT8 attention projection: fp32 activations quantised per token
    inside the call, fused q/k/v weights [3072][1024] (per-channel int8),
    at M = 1 and 16 (decode, 40 rotating weight copies so the weights come
    from HBM) and M = 4096 (prefill)."""
    res = {}
    N, K = 3072, 1024
    copies = 40
    Ws = [api.W8A8(W=torch.randn(N, K, device="cuda") / 32) for _ in range(copies)]
    wbytes = N * K + 4 * N
    for M in (1, 16, 4096):
        X = torch.randn(M, K, device="cuda")
        out = torch.empty(M, N, device="cuda")
        ws = [Ws[0].gemm_f32(X, out, stream=stream)]
        it = [0]

        def step():
            ws[0] = Ws[it[0] % copies].gemm_f32(X, out, ws=ws[0], stream=stream)
            it[0] += 1
        _, ev = time_fn(torch, step, 4 * copies if M <= 16 else 20, copies if M <= 16 else 3,
                        stream)
        assert api.sync_errors(stream) == 0
        r = {"us_per_call": ev * 1e3, "tops": 2.0 * M * N * K / (ev / 1e3) / 1e12,
             "gbps": (wbytes + 4 * M * K + 4 * M * N) / (ev / 1e3) / 1e9}
        r["hbm_frac"] = r["gbps"] * 1e9 / HBM_PEAK
        r["mfma_frac"] = r["tops"] * 1e12 / INT8_PEAK
        res[f"attn_proj_int8_M{M}"] = r
    del Ws
    torch.cuda.empty_cache()
    return res


# the training shape of the reference (bench/kernel/train_tinystories.c:78-81,
# d=64, seq 128 x batch 4) and a layer-sized one
BWD_SHAPES = {"moe_bwd_T512_train": (512, 64, 32, 8, 2, 1),
              "moe_bwd_T4096_layer": (4096, 1024, 256, 64, 8, 1)}
F32_PEAK = 157.3e12   # MI355X fp32 vector (packed FMA)
F32_MULADD = F32_PEAK / 4  # separate, unpacked multiply and add: 1 flop/lane/instruction


def bwd_inputs(np, T, n, h, E, k, S, seed):
    """Synthetic backward inputs (numpy): distinct ids per token, weights in
    (0, 1], caches ~ N(0, 1), the capacity sort at cap 1.25."""
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s, dtype=np.float32)  # noqa
    ids = np.argsort(rng.random((T, E)), axis=1)[:, :k].astype(np.int64)
    cap = int(np.ceil(1.25 * T * k / E))
    flat = ids.ravel()
    drop = np.ones(T * k, np.uint8)
    perm, off = [], [0]
    for e in range(E):
        q = np.nonzero(flat == e)[0][:cap]
        drop[q] = 0
        perm.append(q)
        off.append(off[-1] + q.size)
    c = dict(dY=f(T, n), X=f(T, n), Wgate=f(E, n) / n ** 0.5, Wg=f(E, h, n) / n ** 0.5,
             Wu=f(E, h, n) / n ** 0.5, Wd=f(E, h, n) / h ** 0.5,
             Wg_s=f(S, h, n) / n ** 0.5, Wu_s=f(S, h, n) / n ** 0.5, Wd_s=f(S, h, n) / h ** 0.5,
             ids=ids, w=rng.uniform(0.01, 1.0, (T, k)).astype(np.float32),
             Gsel=f(T * k, h), Usel=f(T * k, h), Ysel=f(T * k, n), Gs=f(T, S, h), Us=f(T, S, h),
             perm=np.concatenate(perm).astype(np.int64), off=np.array(off, np.int64), drop=drop)
    c["Ysel"][drop.astype(bool)] = 0.0
    return c


BWD_ORDER = ("dY", "X", "Wgate", "Wg", "Wu", "Wd", "Wg_s", "Wu_s", "Wd_s", "ids", "w", "Gsel",
             "Usel", "Ysel", "Gs", "Us", "perm", "off", "drop")


def bwd_bench(np, torch, api, stream, T, n, h, E, k, S):
    """jt_hip_moe_bwd_batch with every input resident in HBM (checked form):
    time per call from HIP events on the stream; the fp32 GEMM work is
    6 GEMMs of kept x h x n plus 6 of T x h x n for the shared experts."""
    c = bwd_inputs(np, T, n, h, E, k, S, seed=T + n)
    d = {}
    for key in BWD_ORDER:
        v = c[key]
        dt = torch.int64 if v.dtype == np.int64 else (torch.uint8 if v.dtype == np.uint8
                                                       else torch.float32)
        d[key] = torch.from_numpy(np.ascontiguousarray(v)).to("cuda", dt)
    args = [d[key] for key in BWD_ORDER] + [k]
    rc, out, ws = api.moe_bwd_batch_device(*args, stream=stream)
    assert rc == 0 and api.sync_errors(stream) == 0

    def step():
        r, _, _ = api.moe_bwd_batch_device(*args, out=out, ws=ws, stream=stream)
        assert r == 0
    _, ev = time_fn(torch, step, 10 if T > 1024 else 50, 3, stream)
    assert api.sync_errors(stream) == 0
    kept = int(c["off"][-1])
    flops = 2.0 * 6 * (kept + S * T) * h * n
    del out, ws, d
    torch.cuda.empty_cache()
    return {"ms_per_call": ev, "tokens_per_s": T / (ev / 1e3),
            "shape": dict(T=T, n=n, h=h, E=E, k=k, S=S, cap_factor=1.25, kept=kept),
            "gemm_flop": flops, "gemm_tflops": flops / (ev / 1e3) / 1e12,
            "frac_f32_peak": flops / (ev / 1e3) / F32_PEAK,
            "frac_mul_add_ceiling": flops / (ev / 1e3) / F32_MULADD}


if __name__ == "__main__":
    main()
