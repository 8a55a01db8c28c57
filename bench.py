#!/usr/bin/env python3
"""Benchmark of the circulant attention hot path on one MI355X.

A step is one fused forward + backward of circulant multi-head attention
(circatt_fused_fwd, circatt_fused_bwd_dq, circatt_fused_bwd_dkdv) over one
batch of synthetic N(0,1) float32 inputs already resident in HBM, at the
configuration BASELINE.json's metric is quoted on (cfg3: DotSimilarity,
256x256x64x4, 4 heads, ws = 15).  Prints one JSON line.

Timing: the step is captured once as a HIP graph; it is replayed untimed
back to back for --settle-ms (0.3 s by default: from idle the GPU's clocks
need ~30 ms of sustained load to reach steady state), then W warm-up
replays, then K timed replays (`ms_per_step` and `value`; `--no-graph`
times eager launches instead).  Right after, K eager steps with HIP events
around every entry point give the per-kernel times (`kernels`, roofline).

Roofline: every kernel of the step is priced at its algorithmic FLOPs
(U = 2*P*K*dh*nheads*B per window contraction; forward 2U, dq pass 2U for
dP and dQ, dk/dv pass 2U for dV and dK; recomputation and softmax work not
counted) against MI355X's dense FP32 MFMA peak, 157.3 TFLOP/s.  Kernel times
come from HIP events on the stream the kernels run on.

Inputs: q, k, v, dy drawn on the host in that order from NumPy's PCG64
(seed 1000 + config number: 1003 for cfg3), N(0,1) float32 (ComplexF32:
(re + i im)/sqrt(2)), and copied to the device; the same arrays feed both legs.

cpu_baseline: the oracle's float32 build (oracle/circatt_oracle.c: the
reference's unfused algorithm, OpenMP over all host cores) timed on a bounded
sample of the same workload: the first (head, batch) units of the very inputs
the GPU step uses.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "circulantattention.jl_amd"))

PEAK_FP32_TFLOPS = 157.3  # MI355X dense FP32 (matrix) peak
PEAK_HBM_GBS = 8000.0

CONFIGS = {
    # name: (spatial fastest-first, C, B, nheads, ws, kind, complex)
    "cfg3": ((256, 256), 64, 4, 4, 15, 0, False),
    "cfg4a": ((512, 512), 32, 1, 1, 31, 1, False),
    "cfg4b": ((262144,), 32, 2, 1, 63, 1, False),
    "cfg5": ((320, 320), 32, 2, 2, 11, 0, True),
}


def describe(name):
    dims, C, B, nh, ws, kind, cplx = CONFIGS[name]
    sim = "Distance" if kind else "Dot"
    typ = "ComplexF32" if cplx else "Float32"
    sp = "x".join(str(d) for d in dims)
    return (f"{name}: fused circulant_mh_attention fwd+bwd, {sim}Similarity, {typ}, "
            f"{sp}x{C}x{B}, nheads={nh}, ws={ws}, A not materialised")


SEEDS = {"cfg3": 1003, "cfg4a": 1004, "cfg4b": 1005, "cfg5": 1006}
# the roofline each configuration is reported against: cfg4b (1D, 32
# channels, a window of 63: 63 keys per query against 12 tensor reads and
# writes per pixel) is HBM-bound, the 2D windows are matrix-core bound
BOUND = {"cfg3": "mfma", "cfg4a": "mfma", "cfg4b": "hbm", "cfg5": "mfma"}


def host_inputs(name):
    """q, k, v, dy of the workload, drawn on the host in that order from
    NumPy's PCG64 (the same bits go to the GPU and to the CPU baseline)."""
    import numpy as np

    dims, C, B, nh, ws, kind, cplx = CONFIGS[name]
    rng = np.random.default_rng(SEEDS[name])
    shape = (B, C, *reversed(dims))
    out = []
    for _ in range(4):
        if cplx:
            a = rng.standard_normal(shape, dtype=np.float32) + 1j * rng.standard_normal(
                shape, dtype=np.float32)
            out.append((a / np.sqrt(2)).astype(np.complex64))
        else:
            out.append(rng.standard_normal(shape, dtype=np.float32))
    return out


def cpu_baseline(name, inputs, budget_s=12.0):
    """Time the float32 oracle (reference's unfused algorithm, OpenMP) on
    whole (head, batch) units of the workload's own inputs, in unit order,
    until ~budget_s of CPU work."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))

    import oracle as O

    dims, C, B, nh, ws, kind, cplx = CONFIGS[name]
    dh = C // nh
    P = int(math.prod(dims))

    def unit(a, u):  # head g of batch b, unit g + nh*b (src/attention.jl:44)
        b, g = divmod(u, nh)
        return a[b:b + 1, g * dh:(g + 1) * dh]

    units, total = 0, 0.0
    while units < nh * B and total < budget_s:
        q, k, v, dy = (unit(a, units) for a in inputs)
        t0 = time.perf_counter()
        _, A = O.attention_fwd(kind, q, k, v, ws, 1, precision="f32")
        O.attention_bwd(kind, q, k, v, dy, ws, 1, precision="f32", A=A)
        total += time.perf_counter() - t0
        units += 1
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    pixels = units / nh * P  # one pixel of the metric carries all nh heads
    return {
        "value": pixels / total / 1e6,
        "unit": "Mpixel/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"the first {units} of {nh * B} (head,batch) units of {name}'s own inputs "
                   f"(the GPU step's bits), fwd+bwd of the reference's unfused algorithm "
                   f"(float32 C/OpenMP restatement), {total:.1f} s"),
    }


# Unfused entry points (the Circulant-materialising path), HBM-bound: name ->
# (spatial, C per unit, nb units, ws, complex).  cfg2 is the reference README's
# 128x96x64x2 ws=15 similarity; cfg5's units are its 2 heads x 2 batches of
# ComplexF32 with 16 channels per head (A + m*B and C ⨷ v of README.md:130).
OPS_CONFIGS = {
    "cfg2": ((128, 96), 64, 2, 15, False),
    "cfg5": ((320, 320), 16, 4, 11, True),
    # the large-window configurations (unfused path, windows past 15); only
    # timed when named with --ops-config
    "cfg4a": ((512, 512), 32, 1, 31, False),
    "cfg4b": ((262144,), 32, 2, 63, False),
}
OPS_DEFAULT = ("cfg2", "cfg5")


def bench_ops(args):
    """Time every unfused entry point at the OPS_CONFIGS shapes with HIP events
    on the launch stream; one JSON line per (config, entry point) with the
    algorithmic HBM bytes (each input read once, each output written once) over
    the average launch time against MI355X's 8 TB/s."""
    import torch

    from circulant_attention import _lib as L
    from circulant_attention._functions import ptr

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    g = torch.Generator(device=dev)
    g.manual_seed(2000)
    only_ops = set(filter(None, args.op.split(",")))
    only_cfg = set(filter(None, args.ops_config.split(","))) or set(OPS_DEFAULT)
    for name, (dims, C, nb, ws, cplx) in OPS_CONFIGS.items():
        if name not in only_cfg:
            continue
        nsp = len(dims)
        n1, n2 = dims[0], (dims[1] if nsp == 2 else 1)
        P = int(math.prod(dims))
        K = ws ** nsp
        nnz = P * K * nb
        dt = L.C32 if cplx else L.F32
        dtype = torch.complex64 if cplx else torch.float32
        shape = (nb, C, *reversed(dims))
        x, y, z, dx, dy = (torch.randn(shape, device=dev, dtype=dtype, generator=g)
                           for _ in range(5))
        T = x.numel() * x.element_size()
        A, B, Z = (torch.rand((nb, P, K), device=dev, generator=g) for _ in range(3))
        rowptr = torch.empty((nb, P + 1), device=dev, dtype=torch.int32)
        colval = torch.empty((nb, P * K), device=dev, dtype=torch.int32)
        sums = torch.empty((nb, P), device=dev)
        m = torch.randn(nb, device=dev, generator=g)
        s = 1.0 / math.sqrt(C)
        ops = [
            ("pattern", 4 * (P + 1) * nb + 4 * nnz,
             lambda: L.lib.circatt_pattern(nsp, n1, n2, ws, nb, ptr(rowptr), ptr(colval), sp)),
            ("similarity_dot", 2 * T + 4 * nnz,
             lambda: L.lib.circatt_similarity(L.DOT, dt, nsp, n1, n2, ws, C, nb, s, ptr(x),
                                              ptr(y), ptr(A), sp)),
            ("softmax", 8 * nnz,
             lambda: L.lib.circatt_softmax(K, P * nb, ptr(A), ptr(Z), sp)),
            ("softmax_bwd", 12 * nnz,
             lambda: L.lib.circatt_softmax_bwd(K, P * nb, ptr(A), ptr(B), ptr(Z), sp)),
            ("apply", 4 * nnz + 2 * T,
             lambda: L.lib.circatt_apply(0, dt, nsp, n1, n2, ws, C, nb, ptr(A), ptr(x), ptr(z),
                                         sp)),
            ("apply_transposed", 4 * nnz + 2 * T,
             lambda: L.lib.circatt_apply(1, dt, nsp, n1, n2, ws, C, nb, ptr(A), ptr(x), ptr(z),
                                         sp)),
            ("similarity_bwd_dot", 4 * nnz + 4 * T,
             lambda: L.lib.circatt_similarity_bwd(L.DOT, dt, nsp, n1, n2, ws, C, nb, s, ptr(B),
                                                  ptr(x), ptr(y), ptr(dx), ptr(dy), sp)),
            ("similarity_bwd_distance", 4 * nnz + 4 * T,
             lambda: L.lib.circatt_similarity_bwd(L.DISTANCE, dt, nsp, n1, n2, ws, C, nb, s,
                                                  ptr(B), ptr(x), ptr(y), ptr(dx), ptr(dy), sp)),
            ("rowsum", 4 * nnz + 4 * P * nb,
             lambda: L.lib.circatt_rowsum(nsp, n1, n2, ws, nb, ptr(A), ptr(sums), sp)),
            ("colsum", 4 * nnz + 4 * P * nb,
             lambda: L.lib.circatt_colsum(nsp, n1, n2, ws, nb, ptr(A), ptr(sums), sp)),
            ("axpby_scaled", 12 * nnz,  # C = A + m*B, m per (head, batch)
             lambda: L.lib.circatt_axpby(P * K, nb, None, 1.0, ptr(A), ptr(m), 0.0, ptr(B),
                                         ptr(Z), sp)),
        ]
        for op, nbytes, f in ops:
            if only_ops and op not in only_ops:
                continue
            for _ in range(args.warmup):
                L.check(f())
            torch.cuda.synchronize()
            evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in range(args.steps)]
            for e0, e1 in evs:
                e0.record(stream)
                L.check(f())
                e1.record(stream)
            torch.cuda.synchronize()
            ts = sorted(e0.elapsed_time(e1) for e0, e1 in evs)
            avg = sum(ts) / len(ts)
            gbs = nbytes / (avg / 1e3) / 1e9
            print(json.dumps({
                "op": op, "config": name, "spatial": list(dims), "C": C, "nb": nb, "ws": ws,
                "dtype": "c32" if cplx else "f32", "nnz": nnz, "avg_us": round(avg * 1e3, 2),
                "min_us": round(ts[0] * 1e3, 2), "alg_bytes": nbytes,
                "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                             "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4)}}), flush=True)
        del x, y, z, dx, dy, A, B, Z, rowptr, colval
        torch.cuda.empty_cache()
    if args.calib_copy_mib > 0:
        calib_copy(args.calib_copy_mib)


def calib_copy(mib):
    """torch's device copy of `mib` MiB, three times: a kernel of known HBM
    traffic that scales the FETCH_SIZE / WRITE_SIZE counters."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.randn(n, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    return n * 4


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--settle-ms", type=float, default=300.0,
                    help="untimed back-to-back steps before the warm-up steps, in ms of wall "
                         "time (the GPU's clocks ramp over the first ~30 ms of sustained load)")
    ap.add_argument("--config", default="cfg3", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--math", choices=("split_f16", "f32"), default=None,
                    help="arithmetic of the fused kernels' matrix products (default: the "
                         "library's default, split_f16)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="after the timed region, run 3 device copies of this many MiB "
                         "(reference kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--no-graph", action="store_true",
                    help="time eager launches only (default: the step is also captured as a HIP "
                         "graph, and `value` comes from its replays)")
    ap.add_argument("--ops", action="store_true",
                    help="instead of the fused step, time each unfused entry point (similarity, "
                         "softmax, apply, sums, axpby, pattern) at the cfg2 / cfg5 shapes and "
                         "print one JSON line per entry point (GB/s against HBM peak)")
    ap.add_argument("--op", default="",
                    help="with --ops: comma-separated entry points to time (default: all)")
    ap.add_argument("--ops-config", default="",
                    help="with --ops: comma-separated shapes to time (cfg2, cfg5, cfg4a, cfg4b; "
                         "default: cfg2,cfg5)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the (head, batch) units "
                                   "would shard across GPUs without communication, one slice of "
                                   "nheads*B per GPU"}))
        sys.exit(2)
    if args.ops:
        bench_ops(args)
        return

    import torch

    from circulant_attention import _lib as L
    from circulant_attention._functions import ptr

    if args.math is not None:
        L.check(L.lib.circatt_set_math(L.MATH_F32 if args.math == "f32" else L.MATH_SPLIT_F16))
    math_mode = {L.MATH_SPLIT_F16: "split_f16", L.MATH_F32: "f32"}[L.lib.circatt_get_math()]
    base = json.load(open(os.path.join(ROOT, "BASELINE.json")))
    dims, C, B, nh, ws, kind, cplx = CONFIGS[args.config]
    nsp = len(dims)
    n1, n2 = dims[0], (dims[1] if nsp == 2 else 1)
    P = int(math.prod(dims))
    K = ws ** nsp
    dh = C // nh
    dev = torch.device("cuda:0")
    host = host_inputs(args.config)
    q, k, v, dy = (torch.from_numpy(a).to(dev) for a in host)
    torch.cuda.synchronize()
    y = torch.empty_like(q)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    lse = torch.empty((B * nh, P), device=dev, dtype=torch.float32)
    wbytes = L.lib.circatt_fused_bwd_workspace_bytes(nsp, n1, n2, nh, B)
    work = torch.empty((wbytes // 4,), device=dev, dtype=torch.float32)
    dt = L.C32 if cplx else L.F32
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)

    def fwd(s):
        L.check(L.lib.circatt_fused_fwd(kind, dt, nsp, n1, n2, ws, C, nh, B, ptr(q), ptr(k),
                                        ptr(v), ptr(y), ptr(lse), s))

    def bwd_dq(s):
        L.check(L.lib.circatt_fused_bwd_dq(kind, dt, nsp, n1, n2, ws, C, nh, B, ptr(q), ptr(k),
                                           ptr(v), ptr(y), ptr(dy), ptr(lse), ptr(dq),
                                           ptr(work), wbytes, s))

    def bwd_dkdv(s):
        L.check(L.lib.circatt_fused_bwd_dkdv(kind, dt, nsp, n1, n2, ws, C, nh, B, ptr(q), ptr(k),
                                             ptr(v), ptr(dy), ptr(lse), ptr(dk), ptr(dv),
                                             ptr(work), wbytes, s))

    kernels = [("fwd", fwd), ("bwd_dq", bwd_dq), ("bwd_dkdv", bwd_dkdv)]
    for _, f in kernels:  # first launches (code objects, kernel attributes)
        f(sp)
    torch.cuda.synchronize()

    # the step (the same three entry points) captured once as a HIP graph, as a
    # training loop would launch it; the entry points allocate nothing and
    # record no memset, so they capture
    graph = None
    if not args.no_graph:
        cs = torch.cuda.Stream(dev)
        csp = ctypes.c_void_p(cs.cuda_stream)
        graph = torch.cuda.CUDAGraph()
        cs.wait_stream(stream)
        with torch.cuda.graph(graph, stream=cs):
            for _, f in kernels:
                f(csp)
        torch.cuda.synchronize()

    def step():
        if graph is not None:
            graph.replay()
        else:
            for _, f in kernels:
                f(sp)

    # Settle: from idle, the GPU's clocks need some 20-30 ms of sustained load
    # to reach steady state (cfg3 from idle: the first 25 steps take 740 us on
    # average, steady state 630 us), so before the W warm-up steps the step
    # runs untimed, back to back, for --settle-ms.
    settle_steps = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < args.settle_ms / 1e3:
        for _ in range(10):
            step()
        settle_steps += 10
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # timed region: K steps, synchronised on both sides
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps

    # per-kernel times for the roofline, right after (the clocks still at
    # steady state): K eager steps with HIP events around every launch on the
    # stream the kernels run on
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in kernels] for _ in range(args.steps)]
    t0 = time.perf_counter()
    for s in range(args.steps):
        for (_, f), (e0, e1) in zip(kernels, evs[s]):
            e0.record(stream)
            f(sp)
            e1.record(stream)
    torch.cuda.synchronize()
    ms_step_eager = (time.perf_counter() - t0) * 1e3 / args.steps
    kern_ms = {name: sum(evs[s][i][0].elapsed_time(evs[s][i][1]) for s in range(args.steps)) /
               args.steps for i, (name, _) in enumerate(kernels)}

    mpix = B * P / (ms_step / 1e3) / 1e6
    cfac = 2 if cplx else 1
    U = 2.0 * P * K * dh * nh * B * cfac
    flops = {"fwd": 2 * U, "bwd_dq": 2 * U, "bwd_dkdv": 2 * U}
    kern = {n: {"avg_ms": kern_ms[n], "alg_gflop": flops[n] / 1e9,
                "tflops": flops[n] / (kern_ms[n] / 1e3) / 1e12} for n in kern_ms}
    # algorithmic HBM bytes per launch: T = one q-sized tensor, L = lse or D
    Tb = 4.0 * B * P * C * cfac
    Lb = 4.0 * B * nh * P
    alg_bytes = {"fwd": 4 * Tb + Lb, "bwd_dq": 6 * Tb + 2 * Lb, "bwd_dkdv": 6 * Tb + 2 * Lb}
    for n in kern:
        kern[n]["alg_gb"] = alg_bytes[n] / 1e9
        kern[n]["gbs"] = alg_bytes[n] / (kern_ms[n] / 1e3) / 1e9
    dom = max(kern_ms, key=kern_ms.get)
    achieved = kern[dom]["tflops"]
    traffic, traffic_src = None, None
    tfile = os.path.join("profiles", f"traffic_{args.config}.json")
    if os.path.exists(os.path.join(ROOT, tfile)):
        traffic = json.load(open(os.path.join(ROOT, tfile))).get(dom)
        traffic_src = (f"{tfile}: HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE and "
                       f"WRITE_SIZE runs (not measured in this run)")
    # BASELINE.json's metric names cfg3's shape; the other configurations get
    # the same metric worded for their own
    metric = base["metric"]
    if args.config != "cfg3":
        shape = (f"{dims[0]}²" if len(dims) == 2 and dims[0] == dims[1]
                 else "×".join(str(d) for d in dims))
        metric = (f"CircAtt fwd+bwd Mpixel/s ({shape}×{C}{' complex' if cplx else ''}, ws={ws}, "
                  f"{nh} heads, B={B}); % of roofline")
    out = {
        "metric": metric,
        "value": round(mpix, 3),
        "unit": "Mpixel/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "timing": ("HIP graph of the step's three entry points, replayed" if graph
                   is not None else "eager launches"),
        "settle_ms": args.settle_ms,
        "settle_steps": settle_steps,
        "ms_per_step_eager": round(ms_step_eager, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "c32" if cplx else "f32",
        "math": math_mode,
        "data": f"synthetic N(0,1), NumPy PCG64 seed {SEEDS[args.config]}, resident in HBM",
        "config": {"workload": describe(args.config), "spatial": list(dims), "C": C, "B": B,
                   "nheads": nh, "ws": ws, "similarity": "Distance" if kind else "Dot"},
        "roofline": ({"bound": "mfma", "kernel": dom, "achieved": round(achieved, 3),
                      "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                      "frac": round(achieved / PEAK_FP32_TFLOPS, 4), "traffic": traffic,
                      "traffic_source": traffic_src}
                     if BOUND[args.config] == "mfma" else
                     {"bound": "hbm", "kernel": dom, "achieved": round(kern[dom]["gbs"], 1),
                      "peak": PEAK_HBM_GBS, "unit": "GB/s",
                      "frac": round(kern[dom]["gbs"] / PEAK_HBM_GBS, 4), "traffic": traffic,
                      "traffic_source": traffic_src,
                      "alg_bytes": "fwd 4T + L, each backward pass 6T + 2L (T: one q-sized tensor, "
                                   "L: lse or D)"}),
        "step_hbm": {"alg_mb_per_step": round((12 * Tb + 4 * Lb) / 1e6, 1),
                     "achieved_gbs": round((12 * Tb + 4 * Lb) / (ms_step / 1e3) / 1e9, 1),
                     "frac": round((12 * Tb + 4 * Lb) / (ms_step / 1e3) / 1e9 / PEAK_HBM_GBS, 4)},
        "step_roofline": {"alg_tflop_per_step": 6 * U / 1e12,
                          "achieved_tflops": round(6 * U / (ms_step / 1e3) / 1e12, 3),
                          "frac": round(6 * U / (ms_step / 1e3) / 1e12 / PEAK_FP32_TFLOPS, 4),
                          "ceiling_mpixel_s": round(B * P / (6 * U / (PEAK_FP32_TFLOPS * 1e12))
                                                    / 1e6, 1)},
        "kernels": {n: {kk: round(vv, 4) for kk, vv in d.items()} for n, d in kern.items()},
    }
    if args.calib_copy_mib > 0:
        out["calib_copy_bytes"] = calib_copy(args.calib_copy_mib)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.config, host)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
