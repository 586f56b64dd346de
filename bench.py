"""Benchmark of the gfx950 FP8 block-scale MoE layer
`moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048` on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cpu] [--no-peaks]

A step is one call of the layer (routing, permutation, GEMM1 + SwiGLU, GEMM2,
combine) on one batch of synthetic inputs already resident in HBM.  The
headline workload is timed for exactly K steps between two device
synchronisations.  Every workload in the sweep is also timed
  * from a captured HIP graph of 8 calls, replayed back to back (the device
    time of a call, free of the Python launch path -- the per-workload
    latency),
  * as the reference harness does (moe/scripts/run_local.py:33: warmup 3,
    100 Python-launched iterations, 5 trials, median trial mean),
  * per stage, with hipEvents the library records on its launch stream,
and its CPU reference is timed once on the host cores.  Expert weights rotate
over 4 copies (5.6 GB), continuously across every loop, so that no call finds
its weights in the 256 MB MALL / L2 left by the previous one.

Prints ONE JSON line on stdout (progress goes to stderr).
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

H, I, E_LOCAL, TOP_K = 7168, 2048, 32, 8
STAGES = ("route", "gemm1_swiglu", "gemm2", "combine")
# Algorithmic work (bytes that must cross HBM once, flops of the matmuls).
BYTES_PER_EXPERT = 44_050_944      # fp8 W13 + W2 (44,040,192) + fp32 block scales (10,752)
BYTES_PER_TOKEN = 22_752           # hidden 7168 + scales 224 + logits 1024 + bf16 out 14336
BYTES_BIAS = 512
FLOPS_PER_PAIR = 88_080_384        # 2*7168*4096 + 2*2048*7168
G1_FLOPS_PER_PAIR = 2 * H * 2 * I  # 58,720,256
G2_FLOPS_PER_PAIR = 2 * I * H      # 29,360,128
G1_BYTES_PER_EXPERT = 2 * I * H + 32 * 56 * 4   # 29,367,296
G2_BYTES_PER_EXPERT = H * I + 56 * 16 * 4       # 14,683,648
HBM_PEAK = 8.0e12                  # B/s, MI355X HBM3E
PEAK = {"fp8": 5.0e15, "bf16": 2.5e15}  # dense MFMA FLOP/s
PEAK_CLOCK_GHZ = 2.4                # MI355X peak engine clock the MFMA peaks are quoted at
STAGE_MFMA_DTYPE = {"gemm1_swiglu": "fp8", "gemm2": "bf16"}
GPU_WORKLOADS = ("decode_t1", "decode_t1_s3", "small_t64", "prefill_t1024", "skewed_t8192")
DEFAULT_WORKLOAD = "skewed_t8192"
WEIGHT_COPIES = 4


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def stage_work(stage, T, n_sel, a_act):
    """(algorithmic bytes, flops, peak FLOP/s) of one launch of a stage."""
    # bytes: weights and scales once, token rows once, intermediates once each
    # way (act: bf16 hi + lo = 4 B per value; GEMM2 rows: fp32, or for T <= 64
    # the bf16 output written by GEMM2 itself)
    if stage == "gemm1_swiglu":
        return (a_act * G1_BYTES_PER_EXPERT + T * (H + 56 * 4) + n_sel * I * 4,
                n_sel * G1_FLOPS_PER_PAIR, PEAK["fp8"])
    if stage == "gemm2":
        rows_out = T * H * 2 if T <= 64 else n_sel * H * 4
        return (a_act * G2_BYTES_PER_EXPERT + n_sel * I * 4 + rows_out,
                n_sel * G2_FLOPS_PER_PAIR, PEAK["bf16"])
    if stage == "route":
        return (T * 256 * 4 + 512 + T * TOP_K * 16, 0, None)
    return (n_sel * H * 4 + T * TOP_K * 8 + T * H * 2, 0, None)


def roofline(bytes_, flops, peak_flops, seconds):
    t_hbm = bytes_ / HBM_PEAK
    t_mfma = flops / peak_flops if peak_flops else 0.0
    if t_mfma > t_hbm:
        return {"bound": "mfma", "achieved": flops / seconds / 1e12, "peak": peak_flops / 1e12,
                "unit": "TFLOP/s", "frac": t_mfma / seconds}
    return {"bound": "hbm", "achieved": bytes_ / seconds / 1e9, "peak": HBM_PEAK / 1e9,
            "unit": "GB/s", "frac": t_hbm / seconds}


class Workload:
    def __init__(self, pkg, torch, name, dev, weights_cache):
        self.pkg, self.torch, self.name = pkg, torch, name
        self.cfg = pkg.synth.CONFIGS[name]
        self.T = self.cfg.T
        seed = self.cfg.seed
        if seed not in weights_cache:
            log(f"[bench] generating weights seed={seed} x{WEIGHT_COPIES}")
            base = pkg.synth.weights(seed, dev)
            weights_cache[seed] = [base] + [tuple(t.clone() for t in base) for _ in range(WEIGHT_COPIES - 1)]
        self.w = weights_cache[seed]
        self.tok = pkg.synth.tokens(self.cfg, dev)
        self.out = torch.empty((self.T, H), dtype=torch.bfloat16, device=dev)
        self.k = 0  # calls so far: the weight copy rotates with every call, across all loops

    def call(self, events=None):
        c = self.cfg
        w = self.w[self.k % len(self.w)]
        self.k += 1
        self.pkg.run(*self.tok, *w, c.local_expert_offset, c.routed_scaling_factor, self.out, stage_events=events)

    def counts(self):
        ws = self.pkg.workspace(self.out.device, self.T)
        off = self.pkg.intermediates(ws, self.T).expert_off.cpu().tolist()
        n_sel = off[E_LOCAL]
        a_act = sum(1 for e in range(E_LOCAL) if off[e + 1] > off[e])
        return n_sel, a_act


def time_steps(torch, wl, steps, warmup):
    for _ in range(warmup):
        wl.call()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        wl.call()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def harness_protocol(torch, wl, iters, trials, warmup):
    """hipEvent-timed trials of Python-launched calls on the launch stream;
    returns (median trial mean ms, all)."""
    s = torch.cuda.current_stream()
    for _ in range(warmup):
        wl.call()
    means = []
    for _ in range(trials):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(s)
        for _ in range(iters):
            wl.call()
        b.record(s)
        b.synchronize()
        means.append(a.elapsed_time(b) / iters)
    means.sort()
    return means[len(means) // 2], means


GRAPH_CALLS = 2 * WEIGHT_COPIES  # calls per captured graph: every weight copy twice


def graph_latency(torch, wl, replays, trials):
    """Device time of one call: GRAPH_CALLS calls (rotating weight copies)
    captured in one HIP graph, replayed `replays` times back to back between
    two events; returns (median over trials of ms per call, all trials)."""
    for _ in range(2 * WEIGHT_COPIES):
        wl.call()  # warm: first-use set-up of every copy outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(GRAPH_CALLS):
            wl.call()
    graph.replay()
    torch.cuda.synchronize()
    means = []
    for _ in range(trials):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(replays):
            graph.replay()
        b.record()
        b.synchronize()
        means.append(a.elapsed_time(b) / (replays * GRAPH_CALLS))
    del graph
    means.sort()
    return means[len(means) // 2], means


def stage_times(pkg, torch, wl, iters):
    """Mean device time per stage (ms), from events recorded by the library on
    the stream it launches on."""
    nst = len(STAGES) + 1
    pool = pkg._lib.EventPool(nst * iters)
    try:
        for i in range(iters):
            wl.call(events=pool.ptr(i * nst))
        torch.cuda.synchronize()
        tot = [0.0] * len(STAGES)
        for i in range(iters):
            for s in range(len(STAGES)):
                tot[s] += pool.elapsed_ms(i * nst + s, i * nst + s + 1)
        return {st: tot[k] / iters for k, st in enumerate(STAGES)}
    finally:
        pool.close()


def near_tie_count(torch, logits, bias, ulps=8):
    """Tokens whose selection boundary (4th vs 5th group score, 8th vs 9th
    expert score among the kept groups) lies within `ulps` fp32 ulps: there
    the expert ids may legitimately differ from the reference's, so the bench
    line reports the count.  fp32 torch on the inputs' device."""
    x = logits.float()
    s = 1.0 / (1.0 + torch.exp(-x))
    sb = s + bias.float().reshape(1, -1)
    T = x.shape[0]
    top2 = sb.view(T, 8, 32).topk(2, dim=2).values.sum(dim=2)
    gs = top2.sort(dim=1, descending=True).values

    def ulp(v):
        v = v.abs()
        return torch.nextafter(v, torch.full_like(v, float("inf"))) - v

    near_g = (gs[:, 3] - gs[:, 4]) <= ulps * ulp(gs[:, 3])
    keep = torch.zeros_like(top2, dtype=torch.bool).scatter_(1, top2.topk(4, dim=1).indices, True)
    cand = sb.masked_fill(~keep.repeat_interleave(32, dim=1), float("-inf"))
    cs = cand.topk(9, dim=1).values
    near_e = (cs[:, 7] - cs[:, 8]) <= ulps * ulp(cs[:, 7])
    return int((near_g | near_e).sum().item())


def measure(pkg, torch, wl, iters, trials, warmup, trace=None):
    """Per-workload figures.  `trace` (live_kernel_times for this workload)
    gives the dominant kernel's duration; without it the event-timed stage
    (which carries a few microseconds of event overhead) stands in."""
    g_ms, g_trials = graph_latency(torch, wl, replays=max(1, iters // GRAPH_CALLS), trials=trials)
    h_ms, h_trials = harness_protocol(torch, wl, iters, trials, warmup)
    st = stage_times(pkg, torch, wl, min(iters, 50))
    n_sel, a_act = wl.counts()
    T = wl.T
    B = a_act * BYTES_PER_EXPERT + T * BYTES_PER_TOKEN + BYTES_BIAS
    F = n_sel * FLOPS_PER_PAIR
    sec = g_ms * 1e-3
    layer = roofline(B, F, PEAK["fp8"], sec)
    if trace and trace.get("stage_us"):
        tst = {k: v * 1e-3 for k, v in trace["stage_us"].items()}
        dom = max(tst, key=lambda k: tst[k])
        dom_ms, src = tst[dom], f"rocprofv3 kernel trace in this run ({trace['calls']} calls)"
    else:
        dom = max(STAGES, key=lambda k: st[k])
        dom_ms, src = st[dom], "hipEvents around the stage on its launch stream"
    kb, kf, kp = stage_work(dom, T, n_sel, a_act)
    kern = roofline(kb, kf, kp, dom_ms * 1e-3)
    kern.update({"kernel": dom, "ms": dom_ms, "ms_source": src, "event_ms": st[dom], "algo_bytes": kb,
                 "algo_flops": kf})
    if kf and dom == "gemm2":
        # the same flops against the dense fp8 peak, the bound the layer's
        # target is stated in (GEMM2 runs on bf16 MFMA: see dtype_detail)
        kern["frac_fp8_peak"] = kf / (dom_ms * 1e-3) / PEAK["fp8"]
    return {
        "workload": wl.name, "T": T, "local_expert_offset": wl.cfg.local_expert_offset, "seed": wl.cfg.seed,
        "n_sel": n_sel, "a_act": a_act, "near_tie_tokens": near_tie_count(torch, wl.tok[0], wl.tok[1]),
        "latency_us": g_ms * 1e3, "latency_source": f"graph replay ({GRAPH_CALLS} calls per graph)",
        "graph_trial_us": [round(x * 1e3, 3) for x in g_trials],
        "harness_us": h_ms * 1e3, "harness_trial_us": [round(x * 1e3, 3) for x in h_trials],
        "tflops": F / sec / 1e12, "gbps": B / sec / 1e9,
        "bound": layer["bound"], "roofline_frac": layer["frac"],
        "stage_us": {k: round(v * 1e3, 3) for k, v in st.items()},
        "trace_stage_us": trace.get("stage_us") if trace else None,
        "trace_kernel_us": trace.get("kernel_us") if trace else None,
        "dominant": kern,
    }


def measured_traffic(workload, stage):
    """HBM bytes per launch of `stage` on `workload` from the committed rocprofv3
    counter summaries (profiles/*.txt lines 'TRAFFIC stage=S workload=W
    fetch_bytes=F write_bytes=B', already scaled by the copy calibration), or
    None when no summary covers it.  Returns (bytes, file name)."""
    import glob

    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.txt"))):
        for line in open(path):
            if not line.startswith("TRAFFIC "):
                continue
            kv = dict(tok.split("=", 1) for tok in line.split()[1:] if "=" in tok)
            if kv.get("stage") == stage and kv.get("workload") == workload:
                return int(kv["fetch_bytes"]) + int(kv["write_bytes"]), os.path.relpath(path, ROOT)
    return None, None


# kernel-name prefix -> bench stage (the layer's kernels only)
_STAGE_OF = (("route", "route"), ("perm", "route"), ("gemm1", "gemm1_swiglu"), ("gemm2", "gemm2"),
             ("combine", "combine"))


CLOCK_MIN_US = 100.0  # shortest dispatch whose GUI_ACTIVE / duration is taken as its clock


def _short_kernel(name):
    import re

    return re.sub(r"^void ", "", name.replace("moe::(anonymous namespace)::", ""))


def parse_pmc(files, counter):
    """One --pmc pass of a --calls-only child (the CSV files it wrote) ->
    ({stage: mean bytes per launch}, {stage: GHz}) or None without the
    calibration copy.  `counter` (FETCH_SIZE or WRITE_SIZE, in KiB per
    dispatch) is scaled so that the pass's last device copy (the 1 GiB
    calibration) moves exactly 1 GiB; a stage's bytes are the mean per
    dispatch of each of its kernels, summed.  GRBM_GUI_ACTIVE rows (summed over
    the 8 XCDs) give each stage's clock, GUI / 8 / duration, for stages whose
    dispatches last CLOCK_MIN_US on average."""
    import csv

    sums, calib, calib_id, gui = {}, None, -1, {}
    for f in files:
        for row in csv.DictReader(open(f)):
            name = row["Kernel_Name"]
            val = float(row["Counter_Value"])
            if row["Counter_Name"] == "GRBM_GUI_ACTIVE":
                short = _short_kernel(name)
                dur_ns = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
                for prefix, stage in _STAGE_OF:
                    if short.startswith(prefix) and dur_ns > 0:
                        gui.setdefault(stage, []).append((dur_ns, val / 8 / dur_ns))
                continue
            if row["Counter_Name"] != counter:
                continue
            if "copyBuffer" in name:  # the last one is the 1 GiB calibration copy
                did = int(row["Dispatch_Id"])
                if did > calib_id:
                    calib_id, calib = did, val
                continue
            short = _short_kernel(name)
            for prefix, stage in _STAGE_OF:
                if short.startswith(prefix):
                    key = (stage, short.split("(")[0])
                    sums.setdefault(key, []).append(val)
    if not calib:
        return None
    scale = 1024.0 * (1048576.0 / calib)  # KiB -> bytes, then the copy's 1 GiB
    per_stage = {}
    for (stage, _), vals in sums.items():  # mean per dispatch, summed over a stage's kernels
        per_stage[stage] = per_stage.get(stage, 0.0) + scale * sum(vals) / len(vals)
    clocks = {stage: round(sum(c for _, c in v) / len(v), 3) for stage, v in gui.items()
              if sum(d for d, _ in v) / len(v) >= CLOCK_MIN_US * 1e3}
    return per_stage, clocks


def live_traffic(workload, timeout_s=180):
    """HBM bytes per launch of every stage of `workload`, measured in this
    bench run: two rocprofv3 --pmc passes (FETCH_SIZE, then WRITE_SIZE; one
    counter group each) over child runs of this script (--calls-only plus a
    1 GiB device copy), each scaled so that the copy reads and writes exactly
    1 GiB.  The FETCH_SIZE pass also collects GRBM_GUI_ACTIVE, which arrives
    summed over the 8 XCDs: / 8 / the dispatch's duration is the shader clock
    the stage's kernels ran at (stages whose dispatches last CLOCK_MIN_US or
    more; a short dispatch's counter window is longer than the dispatch).
    Called before this process touches the GPU.  Returns
    ({stage: bytes}, {stage: GHz}, None) or (None, None, reason)."""
    import glob
    import shutil
    import subprocess
    import tempfile

    if shutil.which("rocprofv3") is None:
        return None, None, "rocprofv3 not found"
    tmp = tempfile.mkdtemp(prefix="moe_bench_pmc_")
    env = dict(os.environ, TMPDIR="/tmp")
    per_stage, clocks = {}, {}
    try:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            out = os.path.join(tmp, counter)
            pmc = [counter, "GRBM_GUI_ACTIVE"] if counter == "FETCH_SIZE" else [counter]
            cmd = ["timeout", "-s", "KILL", str(timeout_s), "rocprofv3", "--pmc", *pmc, "--output-format", "csv",
                   "-d", out, "-o", "pmc", "--", sys.executable, os.path.abspath(__file__), "--no-cpu", "--no-quant",
                   "--no-peaks", "--no-traffic", "--sweep", "", "--workload", workload, "--calls-only", "--steps", "3",
                   "--warmup", "1", "--copy-calib-mib", "1024"]
            log(f"[bench] traffic: rocprofv3 --pmc {' '.join(pmc)} pass on {workload}")
            r = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True)
            files = glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True)
            if not files:
                return None, None, f"rocprofv3 --pmc {counter} wrote no counters (exit {r.returncode})"
            parsed = parse_pmc(files, counter)
            if parsed is None:
                return None, None, f"no calibration copy in the {counter} pass"
            for stage, b in parsed[0].items():
                per_stage[stage] = per_stage.get(stage, 0.0) + b
            clocks.update(parsed[1])
        return {k: int(v) for k, v in per_stage.items()}, clocks, None
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


TRACE_CALLS = 20  # calls per workload in the kernel-trace child run


def split_trace(rows, workloads, calls):
    """Kernel-trace rows (dispatch id, kernel name, ns) of a --trace-calls
    child -> ({workload: {"calls", "stage_us", "kernel_us"}}, None), or (None,
    reason) when the trace does not hold one marked span per workload.  The
    i-th trace_mark_begin .. trace_mark_end span holds the `calls` calls of
    the i-th workload; the layer's kernels inside it are summed per stage (us
    per call) and averaged per kernel."""
    order = list(workloads)
    cur, k = None, 0
    per = {}
    for _, name, ns in sorted(rows):
        if "trace_mark_begin" in name:
            cur = order[k] if k < len(order) else None
            k += 1
            continue
        if "trace_mark_end" in name:
            cur = None
            continue
        if cur is None:
            continue
        short = _short_kernel(name).split("(")[0]
        for prefix, stage in _STAGE_OF:
            if short.startswith(prefix):
                d = per.setdefault(cur, {"kernels": {}, "stages": {}})
                n, tot = d["kernels"].get(short, (0, 0))
                d["kernels"][short] = (n + 1, tot + ns)
                d["stages"][stage] = d["stages"].get(stage, 0) + ns
                break
    if k != len(order):
        return None, f"kernel trace holds {k} workload spans, expected {len(order)}"
    out = {}
    for wname, d in per.items():
        out[wname] = {"calls": calls,
                      "stage_us": {st: round(ns / calls / 1e3, 3) for st, ns in d["stages"].items()},
                      "kernel_us": {kn: round(tot / n / 1e3, 3) for kn, (n, tot) in d["kernels"].items()}}
    return out, None


def live_kernel_times(workloads, timeout_s=300):
    """Mean device duration of each of the layer's kernels per workload,
    measured in this bench run: one rocprofv3 --kernel-trace pass over a
    child run of this script (--trace-calls) that makes TRACE_CALLS plain
    calls per workload between two marker kernels (moe_bench_trace_mark).
    Called before this process touches the GPU.  Returns ({workload:
    {"stage_us": {stage: us per call}, "kernel_us": {kernel: mean us},
    "calls": n}}, None) or (None, reason)."""
    import csv
    import glob
    import shutil
    import subprocess
    import tempfile

    if shutil.which("rocprofv3") is None:
        return None, "rocprofv3 not found"
    tmp = tempfile.mkdtemp(prefix="moe_bench_trace_")
    env = dict(os.environ, TMPDIR="/tmp")
    try:
        cmd = ["timeout", "-s", "KILL", str(timeout_s), "rocprofv3", "--kernel-trace", "--output-format", "csv",
               "-d", tmp, "-o", "kt", "--", sys.executable, os.path.abspath(__file__), "--trace-calls",
               ",".join(workloads)]
        log(f"[bench] kernel times: rocprofv3 --kernel-trace pass over {','.join(workloads)}")
        r = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True)
        files = glob.glob(os.path.join(tmp, "**", "*kernel_trace.csv"), recursive=True)
        if not files:
            return None, f"rocprofv3 --kernel-trace wrote no trace (exit {r.returncode})"
        rows = []
        for f in files:
            for row in csv.DictReader(open(f)):
                rows.append((int(row["Dispatch_Id"]), row["Kernel_Name"], int(row["End_Timestamp"]) -
                             int(row["Start_Timestamp"])))
        return split_trace(rows, workloads, TRACE_CALLS)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def trace_calls(pkg, torch, dev, names):
    """The --trace-calls child: per workload, warm-up calls, then a
    trace_mark_begin dispatch, TRACE_CALLS calls and a trace_mark_end."""
    import ctypes

    B = pkg._lib.bench_lib()
    cache = {}
    for name in names:
        wl = Workload(pkg, torch, name, dev, cache)
        for _ in range(3):
            wl.call()
        torch.cuda.synchronize()
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        assert B.moe_bench_trace_mark(0, stream) == 0
        for _ in range(TRACE_CALLS):
            wl.call()
        assert B.moe_bench_trace_mark(1, stream) == 0
        torch.cuda.synchronize()
        log(f"[bench] traced {TRACE_CALLS} calls of {name}")


def copy_calibration(torch, dev, mib):
    """A plain device copy of known size, for scaling FETCH_SIZE / WRITE_SIZE
    counters of a --pmc run of this script."""
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] copy calibration: {n} bytes read + {n} bytes written per copy, 3 copies")


def cpu_time(pkg, torch, wl, budget_s=5.0):
    """The CPU reference on the whole workload, timed on the host cores: the
    oracle, a plain-C restatement of full-agent-pipeline/references/moe.py
    including its dequantise-all-32-experts step (moe.py:107-118), OpenMP over
    the host's threads.  One untimed warmup call and three timed calls (their
    mean) when a call takes less than `budget_s`; otherwise that first call
    is the only one, and it is timed (a bounded sample: ~26 s at T = 8192).
    Returns (seconds per call, OpenMP threads, calls timed)."""
    import numpy as np

    from oracle import oracle as orc

    L = orc.lib()
    cfg = wl.cfg
    w = wl.w[0]
    host_w = (w[0].view(torch.uint8).cpu().numpy(), w[1].cpu().numpy(), w[2].view(torch.uint8).cpu().numpy(),
              w[3].cpu().numpy())
    tok = wl.tok
    host_t = (tok[0].cpu().numpy(), tok[1].view(torch.int16).cpu().numpy().view(np.uint16),
              tok[2].view(torch.uint8).cpu().numpy(), tok[3].cpu().numpy())
    x = orc.Inputs(*host_t, *host_w, orc.Config(cfg.name, cfg.T, cfg.local_expert_offset, cfg.seed,
                                                 cfg.hot_experts, cfg.hot_add, cfg.routed_scaling_factor))
    t0 = time.perf_counter()
    orc.moe(x, dequant_all=True)
    first = time.perf_counter() - t0
    times = [first]
    if first < budget_s:
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            orc.moe(x, dequant_all=True)
            times.append(time.perf_counter() - t0)
    dt = sum(times) / len(times)
    log(f"[bench] cpu reference {cfg.name}: T={cfg.T} {dt:.2f} s per call ({len(times)} timed"
        f"{', after one warmup' if len(times) > 1 else ''}) on {L.orc_num_threads()} threads")
    return dt, L.orc_num_threads(), len(times)


def measured_peaks(pkg, torch, dev):
    """Roofline denominators measured on this GPU: a streaming read of 4 GiB
    (16-byte nontemporal loads, every byte once) and MFMA loops of the two
    instructions the GEMMs use (operands in registers, 16 waves per CU), with
    fixed operands (short runs) and with random ones (sustained)."""
    import ctypes

    L = pkg._lib.bench_lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count

    def timed(fn, reps=5):
        fn()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            b.synchronize()
            best = min(best, a.elapsed_time(b) * 1e-3)
        return best

    nbytes = 4 << 30
    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(3)
    blocks = cus * 4
    mfma_blocks = 2 * cus  # 16 waves per CU: 8 per CU leave the MFMA pipes 10-15% idle
    sink = torch.empty(max(blocks * 256, mfma_blocks * 512), dtype=torch.float32, device=dev)

    def read():
        rc = L.moe_bench_read_stream(ctypes.c_void_p(buf.data_ptr()), nbytes, ctypes.c_void_p(sink.data_ptr()),
                                     blocks, stream)
        assert rc == 0, f"moe_bench_read_stream: hipError {rc}"

    rd = timed(read)
    del buf
    out = {"hbm_read_GBps": round(nbytes / rd / 1e9, 1)}
    for kind, name, k in ((0, "mfma_fp8_TFLOPs", 128), (1, "mfma_bf16_TFLOPs", 32)):
        iters = 4000
        t = timed(lambda: L.moe_bench_mfma_loop(kind, iters, mfma_blocks, ctypes.c_void_p(sink.data_ptr()), stream))
        flops = mfma_blocks * 8 * iters * 8 * 2 * 16 * 16 * k
        out[name] = round(flops / t / 1e12, 1)
    # Sustained with random operands: back-to-back launches for ~1.5 s per
    # instruction, the median of the second half.  The operands' switching
    # power lowers the clock the chip holds (fixed operands keep ~2.3 GHz),
    # so this is the MFMA rate a GEMM on real data can reach at full issue.
    for kind, name, k, iters in ((2, "mfma_fp8_sustained_random_TFLOPs", 128, 2000),
                                 (3, "mfma_bf16_sustained_random_TFLOPs", 32, 4000)):
        launch = lambda: L.moe_bench_mfma_loop(kind, iters, mfma_blocks, ctypes.c_void_p(sink.data_ptr()), stream)
        events, t0 = [], time.perf_counter()
        while time.perf_counter() - t0 < 1.5 and len(events) < 4000:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            rc = launch()
            assert rc == 0, f"moe_bench_mfma_loop({kind}): hipError {rc}"
            b.record()
            events.append((a, b))
            if len(events) % 64 == 0:
                events[-1][1].synchronize()
        torch.cuda.synchronize()
        ts = sorted(a.elapsed_time(b) * 1e-3 for a, b in events[len(events) // 2:])
        flops = mfma_blocks * 8 * iters * 8 * 2 * 16 * 16 * k
        out[name] = round(flops / ts[len(ts) // 2] / 1e12, 1)
    out["method"] = ("streaming read of 4 GiB, one contiguous chunk per workgroup, 16-byte nontemporal loads; "
                     "MFMA loops of v_mfma_f32_16x16x128_f8f6f4 / "
                     "v_mfma_f32_16x16x32_bf16, 8 independent accumulators per wave, 16 waves per CU "
                     "(lib/libmoe_bench.so, csrc/peaks.hip): fixed operands, best of 5 launches; random "
                     "operands, median launch of the second half of ~1.5 s back to back")
    log(f"[bench] measured peaks: {out}")
    return out


def measure_quantizer(pkg, torch, dev, T, iters=100):
    """The step before the layer (pkg.quantize_hidden): bf16 rows [T, 7168]
    -> e4m3 rows + [56, T] scales.  HBM-bound; algorithmic bytes per call =
    T * (2 * 7168 read + 7168 + 56 * 4 written).  Inputs rotate over enough
    buffers (>= 1 GiB together) that each call reads its rows from HBM, not
    from the 256 MB MALL."""
    copies = max(4, (1 << 30) // (T * H * 2) + 1)
    g = torch.Generator(device="cpu").manual_seed(T)
    base = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    xs = [base.roll(i, 0).contiguous() for i in range(copies)]
    q = torch.empty(T, H, dtype=torch.float8_e4m3fn, device=dev)
    sc = torch.empty(H // 128, T, dtype=torch.float32, device=dev)
    for i in range(3):
        pkg.quantize_hidden(xs[i % copies], q, sc)
    torch.cuda.synchronize()
    # The launches are captured in a graph and replayed, so the events time the
    # kernels back to back rather than the Python wrapper's launch rate (a
    # T = 1024 kernel is shorter than one pass through the wrapper).
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(iters):
            pkg.quantize_hidden(xs[i % copies], q, sc)
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    graph.replay()
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) / iters * 1e3
    del graph
    nbytes = T * (2 * H + H + (H // 128) * 4)
    return {"T": T, "latency_us": round(us, 3), "gbps": round(nbytes / us / 1e3, 1),
            "roofline": {"bound": "hbm", "achieved": round(nbytes / us / 1e3, 1), "peak": HBM_PEAK / 1e9,
                         "unit": "GB/s", "frac": round(nbytes / us / 1e3 / (HBM_PEAK / 1e9), 4)},
            "algo_bytes": nbytes}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=GPU_WORKLOADS)
    ap.add_argument("--sweep", default=",".join(GPU_WORKLOADS),
                    help="comma-separated workloads timed per workload ('' = none)")
    ap.add_argument("--iters", type=int, default=100)
    ap.add_argument("--trials", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU reference timings")
    ap.add_argument("--no-quant", action="store_true", help="skip the activation-quantiser measurement")
    ap.add_argument("--no-peaks", action="store_true", help="skip the measured-peak microbenchmarks")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="also run a plain device copy of this size (for PMC byte calibration)")
    ap.add_argument("--no-traffic", action="store_true",
                    help="take roofline.traffic from the committed counter summaries instead of two live "
                         "rocprofv3 --pmc passes")
    ap.add_argument("--calls-only", action="store_true",
                    help="only the headline's plain calls (no graphs, no events): for rocprofv3 --pmc runs")
    ap.add_argument("--trace-calls", default=None,
                    help="child mode of the kernel-trace pass: marked plain calls of these workloads, nothing else")
    ap.add_argument("--no-kernel-trace", action="store_true",
                    help="take dominant-kernel durations from hipEvents instead of a live rocprofv3 kernel trace")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (the layer is one expert-parallel rank's "
              "shard; no collectives are implemented). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.trace_calls is not None:
        import torch

        pkg = importlib.import_module("mlsys-contest-syfi-fully-agent_amd")
        dev = torch.device("cuda:0")
        torch.cuda.set_device(dev)
        trace_calls(pkg, torch, dev, [s for s in args.trace_calls.split(",") if s])
        return

    # HBM traffic and kernel times first, from child processes, before this
    # process touches the GPU
    live, clocks, live_err = ((None, None, "--no-traffic") if (args.no_traffic or args.calls_only)
                              else live_traffic(args.workload))
    if live_err and not args.calls_only:
        log(f"[bench] traffic: live measurement unavailable ({live_err}); using the committed summaries")
    sweep = [s for s in args.sweep.split(",") if s]
    traced = sweep + ([] if args.workload in sweep else [args.workload])
    ktimes, kt_err = ((None, "--no-kernel-trace") if (args.no_kernel_trace or args.calls_only)
                      else live_kernel_times(traced))
    if kt_err and not args.calls_only:
        log(f"[bench] kernel times: live trace unavailable ({kt_err}); dominant kernels event-timed")
    ktimes = ktimes or {}

    import torch

    pkg = importlib.import_module("mlsys-contest-syfi-fully-agent_amd")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    pkg._lib.moe_lib()  # fails loudly if the HIP library is not built
    cache = {}

    results, wls = {}, {}
    for name in sweep:
        wl = wls[name] = Workload(pkg, torch, name, dev, cache)
        log(f"[bench] {name}: T={wl.T}")
        results[name] = measure(pkg, torch, wl, args.iters, args.trials, args.warmup, ktimes.get(name))
        r = results[name]
        log(f"[bench] {name}: {r['latency_us']:.1f} us (graph; harness protocol {r['harness_us']:.1f} us), "
            f"n_sel={r['n_sel']} a_act={r['a_act']} near-ties={r['near_tie_tokens']} {r['tflops']:.1f} TFLOP/s "
            f"{r['gbps']:.0f} GB/s frac={r['roofline_frac']:.3f} stages={r['stage_us']}")

    head = wls.get(args.workload) or Workload(pkg, torch, args.workload, dev, cache)
    ms = time_steps(torch, head, args.steps, args.warmup)
    log(f"[bench] headline {args.workload}: {ms * 1e3:.1f} us/step over {args.steps} steps")
    if args.calls_only:
        if args.copy_calib_mib:
            copy_calibration(torch, dev, args.copy_calib_mib)
        print(json.dumps({"metric": "MoE layer latency (us) (calls only, for counter runs)", "value": round(ms * 1e3, 3),
                          "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": round(ms, 5), "higher_is_better": False,
                          "config": {"workload": args.workload}}), flush=True)
        return
    hm = results.get(args.workload) or measure(pkg, torch, head, args.iters, args.trials, args.warmup,
                                               ktimes.get(args.workload))

    if args.copy_calib_mib:
        copy_calibration(torch, dev, args.copy_calib_mib)
    quant = {}
    if not args.no_quant:
        for Tq in (1024, 8192):
            quant[f"t{Tq}"] = measure_quantizer(pkg, torch, dev, Tq)
            log(f"[bench] quantize_hidden T={Tq}: {quant[f't{Tq}']['latency_us']:.1f} us "
                f"{quant[f't{Tq}']['gbps']:.0f} GB/s")
    peaks = None if args.no_peaks else measured_peaks(pkg, torch, dev)

    cpu = None
    if not args.no_cpu:
        for name, wl in list(wls.items()) + ([] if args.workload in wls else [(args.workload, head)]):
            sec, threads, calls = cpu_time(pkg, torch, wl)
            if name in results:
                results[name]["cpu_us"] = sec * 1e6
                results[name]["cpu_calls_timed"] = calls
                results[name]["speedup_vs_cpu"] = sec * 1e6 / results[name]["latency_us"]
            if name == args.workload:
                affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None
                how = ("one call (a bounded sample: the whole workload once)" if calls == 1
                       else f"mean of {calls} calls after one warmup")
                cpu = {"value": round(sec * 1e6, 1), "unit": "us", "cores": threads, "kind": "port",
                       "affinity_cores": affinity, "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS"),
                       "sample": (f"{how} of the oracle (plain-C restatement of "
                                  f"full-agent-pipeline/references/moe.py incl. its dequantise-all-32-experts "
                                  f"step) on the whole {name} workload (all {wl.T} tokens), OpenMP over "
                                  f"{threads} host threads; measured, not extrapolated")}

    dom = hm["dominant"]
    if live and dom["kernel"] in live:
        traffic = live[dom["kernel"]]
        traffic_src = ("measured in this run: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes (child runs of "
                       "bench.py --calls-only), each scaled by a 1 GiB device copy in the same pass")
    else:
        traffic, path = measured_traffic(args.workload, dom["kernel"])
        traffic_src = (f"{path}: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE run of this bench, copy-calibrated "
                       f"(not measured in this run: {live_err})") if path else None
    roof = {"bound": dom["bound"], "achieved": round(dom["achieved"], 3), "peak": dom["peak"],
            "unit": dom["unit"], "frac": round(dom["frac"], 4), "traffic": traffic,
            "traffic_source": traffic_src, "kernel": dom["kernel"], "kernel_us": round(dom["ms"] * 1e3, 3),
            "kernel_us_source": dom["ms_source"], "kernel_us_events": round(dom["event_ms"] * 1e3, 3)}
    if live:
        roof["traffic_by_stage"] = live
    if dom["kernel"] == "gemm2" and dom["algo_flops"]:  # (a workload without expert work has none)
        # the activation enters as a bf16 (hi, lo) pair: two bf16 MFMAs per product
        roof["mfma_flops_executed"] = 2 * dom["algo_flops"]
        roof["executed_frac"] = round(2 * dom["frac"], 4)
        # `frac` is against the bf16 peak of the instruction GEMM2 runs on;
        # against the dense fp8 peak the layer's target is stated in:
        roof["frac_fp8_peak"] = round(dom["frac_fp8_peak"], 4)
    if clocks and dom["kernel"] in clocks:
        # The published peaks assume the 2.4 GHz peak engine clock; the
        # dominant kernel's own clock (GRBM_GUI_ACTIVE per XCD over its
        # duration, in the FETCH_SIZE pass) scales the peak it can reach.
        ghz = clocks[dom["kernel"]]
        roof["clock_GHz"] = ghz
        roof["clock_source"] = ("GRBM_GUI_ACTIVE / 8 / dispatch duration, rocprofv3 --pmc FETCH_SIZE GRBM_GUI_ACTIVE "
                                "pass of this run (kernels serialised under counter collection)")
        if dom["unit"] == "TFLOP/s":
            roof["peak_at_clock"] = round(dom["peak"] * ghz / PEAK_CLOCK_GHZ, 1)
            roof["frac_at_clock"] = round(dom["achieved"] / roof["peak_at_clock"], 4)
        roof["clock_by_stage"] = clocks
    if peaks:
        key = {"GB/s": "hbm_read_GBps", "TFLOP/s": "mfma_bf16_TFLOPs" if dom["kernel"] == "gemm2" else "mfma_fp8_TFLOPs"}
        roof["peak_measured"] = peaks[key[dom["unit"]]]
        roof["frac_of_measured_peak"] = round(dom["achieved"] / peaks[key[dom["unit"]]], 4)
        if dom["unit"] == "TFLOP/s":
            sk = "mfma_bf16_sustained_random_TFLOPs" if dom["kernel"] == "gemm2" else "mfma_fp8_sustained_random_TFLOPs"
            roof["peak_sustained_random"] = peaks[sk]
            roof["frac_of_sustained_random_peak"] = round(dom["achieved"] / peaks[sk], 4)
            if dom["kernel"] == "gemm2":
                roof["executed_frac_of_sustained_random_peak"] = round(2 * dom["achieved"] / peaks[sk], 4)

    line = {
        "metric": "MoE layer latency (us) + FP8 TFLOPS / HBM GB/s as % roofline, T=1..8192",
        "value": round(ms * 1e3, 3), "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8",
        "dtype_detail": ("e4m3 x e4m3 MFMA (GEMM1); bf16 MFMA on the activation's (hi, lo) bf16 pair x e4m3 "
                         "weights widened exactly (GEMM2); fp32 accumulate, fp32 GEMM2 rows"),
        "data": "synthetic (seeded generator)",
        "config": {"workload": args.workload, "T": head.T, "local_expert_offset": head.cfg.local_expert_offset,
                   "seed": head.cfg.seed, "hot_experts": list(head.cfg.hot_experts), "hot_bias_add": head.cfg.hot_add,
                   "n_sel": hm["n_sel"], "a_act": hm["a_act"], "parallelism": "single GPU (one EP rank)"},
        "tflops": round(hm["tflops"], 2), "gbps": round(hm["gbps"], 1), "layer_roofline_frac": round(hm["roofline_frac"], 4),
        "roofline": roof,
        "cpu_baseline": cpu,
        "measured_peaks": peaks,
        "upstream_quantizer": quant or None,
        "per_workload": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                         for k, v in results.items()},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
