#!/usr/bin/env python3
"""Benchmark of the verify-path int4 matmuls on one MI355X.

Default line: the 27B-class dense verify-linear sweep at M = 16 -- 64 layers
x {q 5120->5120, k 5120->1024, v 5120->1024, o 5120->5120, gate
5120->17408, up 5120->17408, down 17408->5120}, int4 affine group_size 64,
bf16 activations ~ N(0,1), W ~ N(0, 0.02) quantised on the GPU before
timing.  One step = the 448 verify matmuls of one verify pass, replayed from
a HIP graph (``--no-graph``: eager launches).  All weights (12.1 GB) are
resident in HBM and the pass streams every byte once, so the 256 MB
infinity cache cannot hold the working set.

The JSON line: value = algorithmic GB/s of the step (packed weights + bf16
scales/biases + x + y), us_per_call, the HBM roofline of the dominant kernel
(its launches replayed alone and timed with HIP events on the stream they
run on; ``traffic`` = measured HBM bytes per launch from the rocprofv3
FETCH_SIZE / WRITE_SIZE summary in profiles/, when one exists for this
workload and kernel; ``mfma`` = its algorithmic TFLOP/s against the dense
bf16 peak and the MFMA-busy share from the rocprofv3 counter summary) and a
CPU baseline (the oracle's C restatement on this host's cores, on a bounded
sample: layer 0's seven matmuls).

``configs`` holds the other benchmarked workloads, each with the same
fields: ``single`` ([16,4096]x[4096,4096], weights rotated over a 1 GB
pool), ``9b`` (the 9B-class sweep: 32 layers, hidden 4096), ``27b_m8`` /
``27b_m32`` (the 27B sweep at M = 8 / 32), ``moe`` (40 layers of top-8-of-256
routed experts, hidden 2048, expert width 512) and ``lmhead`` (fused lm_head
[16,5120]x[151936,5120] + greedy accept).  ``--workload X`` prints only X's
line (for profiling runs); ``gdn`` (the GDN rollback pair) and ``copy`` (a
512 MiB device copy that calibrates the traffic counters) exist only that
way.

Every timed graph is first replayed untimed: ``--warmup`` times (default 20)
and for at least WARM_MS of GPU time, so the figures are steady-state ones.
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
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "M=16 int4 verify_qmm µs/call + achieved HBM GB/s (% of peak), 1 GPU"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")
MFMA_FILE = os.path.join(ROOT, "profiles", "mfma.json")
MFMA_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA, MI355X
CPU_LABEL = "own CPU restatement, not MLX (oracle/cpu_qmm.c, OpenMP, fp32 accumulate)"
CPU_SAMPLE_S = 4.0  # seconds of CPU work per configuration's baseline

SHAPES_9B = [("q", 4096, 4096), ("k", 4096, 1024), ("v", 4096, 1024), ("o", 4096, 4096),
             ("gate", 4096, 12288), ("up", 4096, 12288), ("down", 12288, 4096)]
SHAPES_27B = [("q", 5120, 5120), ("k", 5120, 1024), ("v", 5120, 1024), ("o", 5120, 5120),
              ("gate", 5120, 17408), ("up", 5120, 17408), ("down", 17408, 5120)]


def alg_bytes(M, K, N, gs=64, bits=4):
    """Algorithmic HBM bytes of one call: packed W + bf16 scales/biases + x + y."""
    return N * K * bits // 8 + 4 * N * K // gs + 2 * M * K + 2 * M * N


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def make_weights(torch, quantize, K, N, gen, dev, gs=64, bits=4):
    w = torch.randn((N, K), generator=gen, device=dev, dtype=torch.float32) * 0.02
    w_q, s, b = quantize(w, gs, bits, torch.bfloat16)
    del w
    return w_q, s, b


def graph_of(torch, fn):
    """Capture fn() into a HIP graph on a side stream (after one eager run)."""
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        fn()
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    torch.cuda.synchronize()
    return g


# Untimed warm-up of every timed graph: at least the requested replays and at
# least this much sustained GPU time.  Measured on MI355X: the first ~30 ms of
# sustained load after a workload's weights are created run slower (the fused
# lm_head 104.2 us/call after 5 warm-up replays, 91.6 us after 100; the 27B
# sweep 3.712 vs 3.685 ms), so the figures are steady-state ones.
WARM_MS = 50.0


def time_replays(torch, g, reps, warmup=2):
    """ms per replay of graph g, HIP events on the stream replay() launches on,
    after ``warmup`` replays and at least WARM_MS of replays."""
    cur = torch.cuda.current_stream()
    w0 = torch.cuda.Event(enable_timing=True)
    w1 = torch.cuda.Event(enable_timing=True)
    w0.record(cur)
    for _ in range(max(1, warmup)):
        g.replay()
    w1.record(cur)
    torch.cuda.synchronize()
    done = max(1, warmup)
    per = w0.elapsed_time(w1) / done
    if done * per < WARM_MS:
        for _ in range(int((WARM_MS - done * per) / max(per, 1e-3)) + 1):
            g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(cur)
    for _ in range(reps):
        g.replay()
    e1.record(cur)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


# ---------------------------------------------------------------- CPU baseline

def cpu_threads():
    n = len(os.sched_getaffinity(0))
    try:
        n = min(n, int(os.environ.get("OMP_NUM_THREADS", n)))
    except ValueError:
        pass
    return max(1, n)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def _host16(torch, t):
    import numpy as np

    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _host_words(t):
    import numpy as np

    return t.contiguous().cpu().numpy().view(np.uint32)


def _cpu_loop(work, nbytes, what):
    """Run work() (one sample unit of nbytes algorithmic bytes) for about
    CPU_SAMPLE_S seconds after one warm-up; GB/s on this host."""
    work()
    reps, t0 = 0, time.perf_counter()
    while True:
        work()
        reps += 1
        el = time.perf_counter() - t0
        if el >= CPU_SAMPLE_S or reps >= 1000:
            break
    gbs = nbytes * reps / el / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": cpu_threads(), "kind": "port",
            "label": CPU_LABEL,
            "sample": f"{what} x {reps} reps, {el:.1f} s on {cpu_model()}"}


def cpu_loaded():
    from oracle import cpu as ocpu

    try:
        ocpu.load()
        return ocpu
    except OSError as exc:  # not built on this host
        log(f"cpu baseline skipped: {exc}")
        return None


def cpu_baseline_calls(torch, calls, M, what):
    """The oracle C restatement over a list of (x, w_q, s, b, ...) matmuls."""
    ocpu = cpu_loaded()
    if ocpu is None:
        return None
    threads = cpu_threads()
    host = [(_host16(torch, c[0]), _host_words(c[1]), _host16(torch, c[2]), _host16(torch, c[3]))
            for c in calls]
    total = sum(alg_bytes(M, h[0].shape[1], h[1].shape[0]) for h in host)

    def work():
        for args in host:
            ocpu.qmm_bf16(*args, 64, 4, threads)
    return _cpu_loop(work, total, what)


# ---------------------------------------------------------------- reports

def measured_traffic(workload, kernel):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            entry = json.load(f).get(workload, {}).get(kernel)
    except (OSError, ValueError):
        return None
    if not entry:
        return None
    return entry.get("bytes_per_launch")


def mfma_report(workload, kernel, flops, us):
    """MFMA side of a launch: algorithmic FLOP (2·rows·K·N) over its measured
    time against the dense bf16 peak, and the MFMA-busy share that the
    committed rocprofv3 counter pass recorded for the kernel (None if absent)."""
    tflops = flops / (us * 1e-6) / 1e12
    util = None
    try:
        with open(MFMA_FILE) as f:
            util = json.load(f).get(workload, {}).get(kernel, {}).get("util_pct")
    except (OSError, ValueError):
        pass
    return {"flops_per_launch": int(flops), "achieved_tflops": round(tflops, 2),
            "peak_tflops": MFMA_PEAK_TFLOPS, "frac": round(tflops / MFMA_PEAK_TFLOPS, 5),
            "busy_pct_counter": util}


def roofline_of(workload, kernel, nbytes, us, flops, per_kernel=None):
    gbs = nbytes / (us * 1e-6) / 1e9
    r = {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(workload, kernel),
         "kernel": kernel, "bytes_per_launch": int(nbytes), "us_per_launch": round(us, 3)}
    if per_kernel is not None:
        r["per_kernel"] = per_kernel
    r["mfma"] = mfma_report(workload, kernel, flops, us)
    return r


def line(value_gbs, ms, n_calls, config, roofline, cpu=None):
    out = {"value": round(value_gbs, 2), "unit": "GB/s", "ms_per_step": round(ms, 4),
           "us_per_call": round(ms * 1e3 / n_calls, 3),
           "pct_of_hbm_peak": round(100 * value_gbs / HBM_PEAK_GBS, 2),
           "config": config, "roofline": roofline}
    if cpu is not None:
        out["cpu_baseline"] = cpu
    return out


# ---------------------------------------------------------------- workloads

class Sweep:
    """Weights of a dense sweep (built once; reused at every M)."""

    def __init__(self, torch, big, bits):
        from dflash_mlx_amd.quantize import quantize

        self.torch = torch
        self.dev = torch.device("cuda:0")
        self.big = big
        self.bits = bits
        self.shapes = SHAPES_27B if big else SHAPES_9B
        self.layers = 64 if big else 32
        gen = torch.Generator(device=self.dev)
        t0 = time.time()
        self.weights = []
        for l in range(self.layers):
            gen.manual_seed(100 + l)
            for (_, K, N) in self.shapes:
                self.weights.append(make_weights(torch, quantize, K, N, gen, self.dev, bits=bits))
        torch.cuda.synchronize()
        log(f"{'27b' if big else '9b'} weights ready: {len(self.weights)} matrices, "
            f"{time.time() - t0:.1f} s")

    def model(self, fuse):
        """The sweep's verify linears as a module tree -- layer l's q/k/v/o
        under ``self_attn`` and gate/up/down under ``mlp``, sharing the weight
        tensors -- swapped in by ``install_verify_linears`` as the loader does
        (verify kernels on; q/k/v and gate/up grouped unless ``fuse`` is
        False) and prewarmed.  Cached per ``fuse``."""
        cache = self.__dict__.setdefault("_models", {})
        if fuse in cache:
            return cache[fuse]
        from torch import nn

        from dflash_mlx_amd.verify_linear import (QuantizedLinear, install_verify_linears,
                                                  prewarm_verify_kernels)

        names = [("self_attn", "q_proj"), ("self_attn", "k_proj"), ("self_attn", "v_proj"),
                 ("self_attn", "o_proj"), ("mlp", "gate_proj"), ("mlp", "up_proj"),
                 ("mlp", "down_proj")]
        root = nn.Module()
        root.layers = nn.ModuleList()
        for l in range(self.layers):
            layer = nn.Module()
            layer.self_attn, layer.mlp = nn.Module(), nn.Module()
            for i, (par, nm) in enumerate(names):
                w, sc, bi = self.weights[l * len(self.shapes) + i]
                setattr(getattr(layer, par), nm,
                        QuantizedLinear(w, sc, bi, group_size=64, bits=self.bits))
            root.layers.append(layer)
        n = install_verify_linears(root, enable_qmm=True, fuse_siblings=fuse)
        assert n == len(self.weights), n
        prewarm_verify_kernels(root)
        self.torch.cuda.synchronize()
        cache[fuse] = root
        return root

    def drop_models(self):
        self.__dict__.pop("_models", None)

    def calls(self, root, M):
        """The step: per layer ``(x, [modules])`` for q/k/v (one input), o,
        gate/up (one input) and down, each input seeded, as a decoder layer
        calls them."""
        torch = self.torch
        groups = [[0, 1, 2], [3], [4, 5], [6]]
        out = []
        for l, layer in enumerate(root.layers):
            mods = [layer.self_attn.q_proj, layer.self_attn.k_proj, layer.self_attn.v_proj,
                    layer.self_attn.o_proj, layer.mlp.gate_proj, layer.mlp.up_proj,
                    layer.mlp.down_proj]
            for grp in groups:
                i0 = l * len(self.shapes) + grp[0]
                K = self.shapes[grp[0]][1]
                xg = torch.Generator(device=self.dev)
                xg.manual_seed(10000 + i0)
                x = torch.randn((M, K), generator=xg, device=self.dev).to(torch.bfloat16)
                out.append((x, [mods[i] for i in grp]))
        return out


def launch_bytes(M, x, mods, bits):
    """Algorithmic bytes of one launch: every matrix's packed weights, scales
    and biases and output rows, the shared activations once."""
    K = x.shape[1]
    return 2 * M * K + sum(alg_bytes(M, K, m.weight.shape[0], bits=bits) - 2 * M * K
                           for m in mods)


def call_kernel(lib, M, x, mods, bits, fuse):
    """Name of the kernel a step call launches: the grouped siblings' shared
    launch (its pair tables side by side: qmm_stream_fused_kernel), or one
    module's launch."""
    K = x.shape[1]
    st = mods[0].__dict__.get("_verify_state")
    if fuse and len(mods) > 1 and st is not None and st.group is not None:
        grp = st.group
        if grp.fused is not None and len(grp.active) == len(grp.states) and 2 <= len(mods) <= 3:
            return "qmm_stream_fused_kernel"
        ns = (ctypes.c_int64 * len(mods))(*[m.weight.shape[0] for m in mods])
        return lib.dfmi_qmm_multi_kernel_name(M, K, ns, len(mods), 64, bits).decode()
    return lib.dfmi_qmm_kernel_name(M, K, mods[0].weight.shape[0], 64, bits, None).decode()


def run_sweep(args, torch, sweep, M, name, with_cpu=True, fuse=True, also_eager=False):
    """One sweep line: graph replays of the step's module calls (eager calls
    with --no-graph).  The modules are the drop-in path: installed verify
    linears, siblings grouped into shared-activation launches unless fuse is
    False.  also_eager: time the eager calls too and report them beside."""
    from dflash_mlx_amd import _lib

    bits = sweep.bits
    lib = _lib.load()
    root = sweep.model(fuse)
    calls = sweep.calls(root, M)
    step_bytes = sum(launch_bytes(M, x, mods, bits) if fuse else
                     sum(launch_bytes(M, x, [m], bits) for m in mods) for (x, mods) in calls)
    n_launches = len(calls) if fuse else sum(len(mods) for (_, mods) in calls)

    def step_of(subset):
        def fn():
            for (x, mods) in subset:
                for m in mods:
                    m(x)
        return fn

    def eager_ms():
        stream = torch.cuda.Stream()
        step = step_of(calls)
        with torch.cuda.stream(stream):
            for _ in range(args.warmup):
                step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        with torch.cuda.stream(stream):
            for _ in range(args.steps):
                step()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps

    eager = args.no_graph
    other_ms = None
    if eager:
        ms = eager_ms()
    else:
        g = graph_of(torch, step_of(calls))
        ms = time_replays(torch, g, args.steps, warmup=args.warmup)
        del g
        if also_eager:
            other_ms = eager_ms()
    log(f"{name}: {ms:.3f} ms/step ({n_launches} launches"
        f"{', eager' if eager else ', graph replays'})")
    gbs = step_bytes / (ms * 1e-3) / 1e9

    # each kernel's launches replayed alone
    groups = {}
    for (x, mods) in calls:
        units = [mods] if fuse else [[m] for m in mods]
        for u in units:
            groups.setdefault(call_kernel(lib, M, x, u, bits, fuse), []).append((x, u))
    per_kernel = {}
    reps = max(3, args.steps // 4)
    for kname, subset in groups.items():
        gk = graph_of(torch, step_of(subset))
        kms = time_replays(torch, gk, reps)
        del gk
        kbytes = sum(launch_bytes(M, x, mods, bits) for (x, mods) in subset)
        kflops = sum(2 * M * x.shape[1] * m.weight.shape[0] for (x, mods) in subset
                     for m in mods)
        per_kernel[kname] = {"launches_per_step": len(subset), "ms_per_step": round(kms, 4),
                             "us_per_launch": round(kms * 1e3 / len(subset), 3),
                             "bytes_per_launch": kbytes // len(subset),
                             "flops_per_launch": kflops // len(subset),
                             "GBps": round(kbytes / (kms * 1e-3) / 1e9, 2)}
    dom = max(per_kernel, key=lambda k: per_kernel[k]["ms_per_step"])
    d = per_kernel[dom]
    wl = ("27b" if sweep.big else "9b") + ("" if M == 16 else f"_m{M}") + \
        ("_bits8" if bits == 8 else "")
    roofline = roofline_of(wl, dom, d["bytes_per_launch"], d["us_per_launch"],
                           d["flops_per_launch"], per_kernel)
    config = {"workload": f"{'27b' if sweep.big else '9b'}-class dense verify-linear sweep",
              "layers": sweep.layers, "linears_per_layer": len(sweep.shapes), "M": M,
              "group_size": 64, "bits": bits,
              "launch": ("eager module calls" if eager else "hip-graph replays of the module calls") +
                        (" (install_verify_linears default: q/k/v and gate/up each one "
                         "shared-activation launch)" if fuse
                         else " (fuse_siblings=False: one launch per matmul)"),
              "launches_per_step": n_launches, "algorithmic_bytes_per_step": step_bytes}
    if other_ms is not None:
        config["eager_ms_per_step"] = round(other_ms, 4)
    cpu = None
    if with_cpu and not args.no_cpu and bits == 4:
        layer0 = [(x, m.weight, m.scales, m.biases) for (x, mods) in calls[:4] for m in mods]
        cpu = cpu_baseline_calls(torch, layer0, M,
                                 f"layer 0 of the sweep ({len(sweep.shapes)} matmuls, M={M})")
    del calls
    return line(gbs, ms, len(sweep.weights), config, roofline, cpu)


def run_single(args, torch):
    from dflash_mlx_amd import _lib
    from dflash_mlx_amd.quantize import quantize
    from dflash_mlx_amd.verify_qmm import qmm_launch

    dev = torch.device("cuda:0")
    M, K, N = args.m if args.workload == "single" else 16, 4096, 4096
    per = N * K // 2 + 4 * N * K // 64
    R = max(2, math.ceil(1.0e9 / per))
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    w_q, s, b = make_weights(torch, quantize, K, N, gen, dev)
    pool = [(w_q, s, b)] + [(w_q.clone(), s.clone(), b.clone()) for _ in range(R - 1)]
    xg = torch.Generator(device=dev)
    xg.manual_seed(0)
    x = torch.randn((M, K), generator=xg, device=dev).to(torch.bfloat16)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    def fn():
        for (wq, sc, bi) in pool:
            qmm_launch(x, wq, sc, bi, N, 64, 4, None, out=y)

    g = graph_of(torch, fn)
    ms = time_replays(torch, g, args.steps, warmup=args.warmup)
    del g
    us = ms * 1e3 / R
    gbs = alg_bytes(M, K, N) / (us * 1e-6) / 1e9
    name = _lib.load().dfmi_qmm_kernel_name(M, K, N, 64, 4, None).decode()
    roofline = roofline_of("single", name, alg_bytes(M, K, N), us, 2 * M * K * N)
    config = {"workload": f"single call [{M},4096]x[4096,4096] int4 gs64, weights rotated over "
                          f"{R} copies (1 GB)", "M": M, "K": K, "N": N}
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_calls(torch, [(x, w_q, s, b)], M, f"one [{M},4096]x[4096,4096] call")
    del pool
    return line(gbs, ms, R, config, roofline, cpu)


def run_lmhead(args, torch):
    import numpy as np

    from dflash_mlx_amd.lm_head import lm_head_greedy_accept
    from dflash_mlx_amd.quantize import quantize

    dev = torch.device("cuda:0")
    M, K, V = 16, 5120, 151936
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    w_q = torch.empty((V, K // 8), dtype=torch.int32, device=dev)
    s = torch.empty((V, K // 64), dtype=torch.bfloat16, device=dev)
    b = torch.empty_like(s)
    for r0 in range(0, V, 16384):  # quantise in row blocks (fp32 W would be 3 GB)
        r1 = min(V, r0 + 16384)
        w = torch.randn((r1 - r0, K), generator=gen, device=dev) * 0.02
        w_q[r0:r1], s[r0:r1], b[r0:r1] = quantize(w, 64, 4, torch.bfloat16)
        del w
    h = torch.randn((M, K), generator=gen, device=dev).to(torch.bfloat16)
    ids = torch.randint(0, V, (M,), generator=gen, device=dev, dtype=torch.int32)
    # six weight copies, each called once per graph replay: 2.6 GB of weights
    # and 292 MB of pair tables, so that neither stays in the 256 MB infinity
    # cache from one call of a head to the next, and the figure is a call's
    # steady-state time rather than one graph launch per call
    R = 6
    heads = [(w_q, s, b)] + [(w_q.clone(), s.clone(), b.clone()) for _ in range(R - 1)]

    def fn():
        for (wq_r, s_r, b_r) in heads:
            lm_head_greedy_accept(h, wq_r, s_r, b_r, verify_ids=ids, group_size=64)

    g = graph_of(torch, fn)
    ms_step = time_replays(torch, g, args.steps, warmup=args.warmup)  # one step = R calls
    del g
    ms = ms_step / R
    nbytes = V * K // 2 + 4 * V * K // 64 + 2 * M * K + 12 * M
    gbs = nbytes / (ms * 1e-3) / 1e9
    roofline = roofline_of("lmhead", "lmhead_stream_kernel", nbytes, ms * 1e3, 2 * M * K * V)
    config = {"workload": "fused lm_head [16,5120]x[151936,5120] int4 gs64 + greedy + accept",
              "M": M, "K": K, "V": V, "calls_per_step": R}
    cpu = None
    ocpu = cpu_loaded() if not args.no_cpu else None
    if ocpu is not None:
        import oracle

        hx, hw, hs, hb = _host16(torch, h), _host_words(w_q), _host16(torch, s), _host16(torch, b)
        hid = ids.cpu().numpy().astype(np.int64)
        threads = cpu_threads()

        def work():
            logits = ocpu.qmm_bf16(hx, hw, hs, hb, 64, 4, threads)
            post = oracle.greedy_tokens_with_mask(logits, dtype="bf16")
            oracle.verify_cycle_accept(hid, post)
        cpu = _cpu_loop(work, nbytes, "one fused lm_head [16,5120]x[151936,5120] + greedy + accept")
    del heads
    return line(gbs, ms_step, R, config, roofline, cpu)


def run_moe(args, torch):
    import numpy as np

    from dflash_mlx_amd.moe import gather_qmm, gather_swiglu, moe_combine
    from dflash_mlx_amd.quantize import quantize

    dev = torch.device("cuda:0")
    T, k, E, D, I, layers = 16, 8, 256, 2048, 512, 40
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)

    def experts(N, K):
        w = torch.randn((E * N, K), generator=gen, device=dev) * 0.02
        wq, sc, bi = quantize(w, 64, 4, torch.bfloat16)
        del w
        return wq.reshape(E, N, K // 8), sc.reshape(E, N, K // 64), bi.reshape(E, N, K // 64)

    lay = []
    total = 0
    sw_bytes = dn_bytes = 0  # algorithmic bytes of the gate/up and the down launches
    per_expert = I * D // 2 + 4 * I * D // 64
    for _ in range(layers):
        gate, up, down = experts(I, D), experts(I, D), experts(D, I)
        logits = torch.randn((T, E), generator=gen, device=dev)
        probs = torch.softmax(logits, dim=-1)
        sc, inds = torch.topk(probs, k, dim=-1)
        sc = (sc / sc.sum(-1, keepdim=True)).float()
        flat = inds.reshape(-1)
        order = torch.argsort(flat, stable=True)
        rhs = flat[order].to(torch.int32)
        lhs = (order // k).to(torch.int32)
        inv = torch.empty_like(order)
        inv[order] = torch.arange(order.numel(), device=dev)
        inv = inv.to(torch.int32)  # row of each pair in the expert-sorted outputs
        n_e = int(torch.unique(flat).numel())
        total += n_e * 3 * per_expert + 2 * T * D * 2
        sw_bytes += n_e * 2 * per_expert + T * D * 2 + T * k * I * 2
        dn_bytes += n_e * per_expert + T * k * I * 2 + T * k * D * 2
        x = torch.randn((T, D), generator=gen, device=dev).to(torch.bfloat16)
        lay.append((gate, up, down, rhs, lhs, inv, sc, x, inds))
    torch.cuda.synchronize()
    log(f"moe weights ready ({layers} layers)")

    def fn():
        for (gate, up, down, rhs, lhs, inv, sc, x, _) in lay:
            h = gather_swiglu(x, gate, up, rhs, lhs_indices=lhs, group_size=64)
            y = gather_qmm(h, *down, rhs, group_size=64)
            moe_combine(y, sc, y_rows=inv)

    g = graph_of(torch, fn)
    ms = time_replays(torch, g, args.steps, warmup=args.warmup)
    gbs = total / (ms * 1e-3) / 1e9
    del g

    # each gather kernel's launches replayed alone (the gate/up SwiGLU pair
    # dominates: two thirds of the weight bytes); both are moe_stream_kernel
    # (pair tables), the SwiGLU and the plain instantiation
    hs = [gather_swiglu(x, gate, up, rhs, lhs_indices=lhs, group_size=64)
          for (gate, up, down, rhs, lhs, inv, sc, x, _) in lay]

    def fn_sw():
        for (gate, up, down, rhs, lhs, inv, sc, x, _) in lay:
            gather_swiglu(x, gate, up, rhs, lhs_indices=lhs, group_size=64)

    def fn_dn():
        for h, (gate, up, down, rhs, lhs, inv, sc, x, _) in zip(hs, lay):
            gather_qmm(h, *down, rhs, group_size=64)

    reps = max(3, args.steps // 4)
    per_kernel = {}
    for name, f, nbytes in (("moe_stream_kernel<swiglu>", fn_sw, sw_bytes),
                            ("moe_stream_kernel<down>", fn_dn, dn_bytes)):
        gk = graph_of(torch, f)
        kms = time_replays(torch, gk, reps)
        del gk
        per_kernel[name] = {"launches_per_step": layers, "ms_per_step": round(kms, 4),
                            "us_per_launch": round(kms * 1e3 / layers, 3),
                            "bytes_per_launch": nbytes // layers,
                            "GBps": round(nbytes / (kms * 1e-3) / 1e9, 2)}
    dom = per_kernel["moe_stream_kernel<swiglu>"]
    # algorithmic FLOP of the gate/up launch: T·k routed rows x (gate + up)
    roofline = roofline_of("moe", "moe_stream_kernel<swiglu>", dom["bytes_per_launch"],
                           dom["us_per_launch"], 2 * T * k * D * I * 2, per_kernel)
    config = {"workload": "MoE 40 layers, 16 tokens top-8 of 256 experts, hidden 2048, "
                          "expert width 512, int4 gs64", "algorithmic_bytes_per_step": total}
    cpu = None
    ocpu = cpu_loaded() if not args.no_cpu else None
    if ocpu is not None:
        from oracle import moe as omoe

        gate, up, down, rhs, lhs, inv, sc, x, inds = lay[0]
        hx = _host16(torch, x)
        hi = inds.cpu().numpy()
        hsc = sc.cpu().numpy()
        host = {}
        for e in np.unique(hi):
            host[int(e)] = tuple((_host_words(t[0][e]), _host16(torch, t[1][e]),
                                  _host16(torch, t[2][e])) for t in (gate, up, down))
        threads = cpu_threads()
        n_e = len(host)
        layer_bytes = n_e * 3 * per_expert + 2 * T * D * 2

        def work():
            y = np.zeros((T * k, D), np.uint16)
            for e, (g_, u_, d_) in host.items():
                pairs = np.nonzero(hi.reshape(-1) == e)[0]
                xr = hx[pairs // k]
                gv = ocpu.qmm_bf16(xr, *g_, 64, 4, threads)
                uv = ocpu.qmm_bf16(xr, *u_, 64, 4, threads)
                h = omoe._silu_mul(gv, uv, "bf16")
                y[pairs] = ocpu.qmm_bf16(h, *d_, 64, 4, threads)
            omoe.moe_combine(y, hsc, dtype="bf16", out_dtype="bf16")
        cpu = _cpu_loop(work, layer_bytes, f"MoE layer 0 ({n_e} distinct experts x gate/up/down "
                                           f"+ SwiGLU + combine)")
    del lay, hs
    return line(gbs, ms, 3 * layers, config, roofline, cpu)


def run_gdn(args, torch):
    """GDN rollback pair of one verify cycle per GDN layer: the recurrence with
    tape over the 16-token block, then the replay of 9 accepted steps, on 64
    layers' worth of distinct fp32 states (the state, 4 MiB per layer, is the
    traffic that bounds both kernels)."""
    from dflash_mlx_amd.gdn import gated_delta_kernel_with_tape, tape_replay_kernel

    dev = torch.device("cuda:0")
    B, T, Hk, Hv, Dk, Dv, layers, acc = 1, 16, 16, 32, 128, 128, 64, 8
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    q = (torch.randn((B, T, Hk, Dk), generator=gen, device=dev) / Dk ** 0.5).to(torch.bfloat16)
    k = (torch.randn((B, T, Hk, Dk), generator=gen, device=dev) / Dk ** 0.5).to(torch.bfloat16)
    v = torch.randn((B, T, Hv, Dv), generator=gen, device=dev).to(torch.bfloat16)
    g = torch.rand((B, T, Hv), generator=gen, device=dev) * 0.15 + 0.85
    beta = torch.rand((B, T, Hv), generator=gen, device=dev).to(torch.bfloat16)
    states = [torch.randn((B, Hv, Dv, Dk), generator=gen, device=dev) * 0.1 for _ in range(layers)]
    tapes = [gated_delta_kernel_with_tape(q, k, v, g, beta, s_)[2] for s_ in states]

    def fn_tape():
        for s_ in states:
            gated_delta_kernel_with_tape(q, k, v, g, beta, s_)

    def fn_replay():
        for s_, t_ in zip(states, tapes):
            tape_replay_kernel(t_[:, :acc + 1], k[:, :acc + 1], g[:, :acc + 1], s_)

    ms_tape = time_replays(torch, graph_of(torch, fn_tape), args.steps, warmup=args.warmup)
    ms_rep = time_replays(torch, graph_of(torch, fn_replay), args.steps, warmup=args.warmup)
    st_bytes = B * Hv * Dv * Dk * 4
    tape_bytes = 2 * st_bytes + 2 * B * T * Hk * Dk * 2 + 2 * B * T * Hv * Dv * 2 \
        + B * T * Hv * Dv * 4 + B * T * Hv * 6
    rep_bytes = 2 * st_bytes + (acc + 1) * (B * Hv * Dv * 4 + B * Hk * Dk * 2 + B * Hv * 4)
    us_tape = ms_tape * 1e3 / layers
    us_rep = ms_rep * 1e3 / layers
    gbs = tape_bytes / (us_tape * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic("gdn", "gdn_kernel<4, false, 0>"),
                "kernel": "gdn_kernel<4, false, 0>", "bytes_per_launch": tape_bytes,
                "us_per_launch": round(us_tape, 3),
                "replay": {"kernel": "gdn_kernel<4, true, 0>", "steps": acc + 1,
                           "bytes_per_launch": rep_bytes, "us_per_launch": round(us_rep, 3),
                           "GBps": round(rep_bytes / (us_rep * 1e-6) / 1e9, 2)}}
    config = {"workload": "GDN rollback pair per layer: gated delta + tape over 16 steps, "
                          "replay of 9 steps; B=1, Hk=16, Hv=32, Dk=Dv=128, fp32 state, 64 layers",
              "T": T, "Hk": Hk, "Hv": Hv, "Dk": Dk, "Dv": Dv}
    return line(gbs, ms_tape, layers, config, roofline)


def run_copy(args, torch):
    """Plain device copy of a known size: calibrates the FETCH_SIZE /
    WRITE_SIZE counters (bytes per dispatch read and written are both
    exactly 512 MiB)."""
    dev = torch.device("cuda:0")
    n = 512 * 1024 * 1024 // 4
    src = torch.ones(n, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    gbs = 2 * n * 4 / (ms * 1e-3) / 1e9
    return {"workload": "copy 512 MiB (counter calibration)", "bytes_read": n * 4,
            "bytes_written": n * 4, "ms_per_copy": round(ms, 4), "GBps_read_plus_write": round(gbs, 1)}


def headline(args, ln):
    """The driver's one-line contract around a workload line."""
    out = {
        "metric": METRIC,
        "value": ln["value"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ln["ms_per_step"],
        "us_per_call": ln["us_per_call"],
        "pct_of_hbm_peak": ln["pct_of_hbm_peak"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights quantised int4 gs64 on GPU)",
        "config": ln["config"],
        "roofline": ln["roofline"],
    }
    if "cpu_baseline" in ln:
        out["cpu_baseline"] = ln["cpu_baseline"]
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="27b",
                    choices=["27b", "9b", "single", "lmhead", "moe", "gdn", "copy"])
    ap.add_argument("--m", type=int, default=16)
    ap.add_argument("--bits", type=int, default=4, choices=[4, 8],
                    help="weight bits of the 9b / 27b sweeps")
    ap.add_argument("--no-graph", action="store_true",
                    help="sweeps: time eager module calls instead of graph replays")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-fuse", action="store_true",
                    help="sweeps: install_verify_linears(fuse_siblings=False), one launch per "
                         "matmul")
    ap.add_argument("--no-configs", action="store_true",
                    help="default run: print the 27B line without the other configurations")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU only (--gpus 1); how the path "
                                   "shards over several GPUs is a design note, not a run"}))
        sys.exit(2)
    import torch

    import __graft_entry__

    __graft_entry__.load_package()
    wl = args.workload
    if wl in ("27b", "9b"):
        sweep = Sweep(torch, wl == "27b", args.bits)
        # graph replays (how a serving loop launches a captured step); the
        # 27B M=16 line also times the same module calls made eagerly
        res = headline(args, run_sweep(args, torch, sweep, args.m, f"{wl} M={args.m}",
                                       fuse=not args.no_fuse,
                                       also_eager=wl == "27b" and args.m == 16))
        default_run = wl == "27b" and args.m == 16 and args.bits == 4 and not args.no_configs
        if default_run:
            configs = {}
            for M in (8, 32):
                configs[f"27b_m{M}"] = run_sweep(args, torch, sweep, M, f"27b M={M}")
            configs["27b_separate"] = run_sweep(args, torch, sweep, 16, "27b M=16 separate",
                                                with_cpu=False, fuse=False, also_eager=True)
            sweep.drop_models()
            del sweep
            torch.cuda.empty_cache()
            configs["9b"] = run_sweep(args, torch, Sweep(torch, False, 4), 16, "9b M=16")
            torch.cuda.empty_cache()
            configs["single"] = run_single(args, torch)
            torch.cuda.empty_cache()
            configs["moe"] = run_moe(args, torch)
            torch.cuda.empty_cache()
            configs["lmhead"] = run_lmhead(args, torch)
            res["configs"] = configs
    elif wl == "copy":
        res = run_copy(args, torch)
    else:
        res = headline(args, {"single": run_single, "lmhead": run_lmhead, "moe": run_moe,
                              "gdn": run_gdn}[wl](args, torch))
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
