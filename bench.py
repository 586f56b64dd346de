"""Benchmark of the gfx950 FP8 block-scale MoE layer
`moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048` on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cpu]

A step is one call of the layer (routing, permutation, GEMM1 + SwiGLU, GEMM2,
combine) on one batch of synthetic inputs already resident in HBM.  The
headline workload is timed for exactly K steps between two device
synchronisations; every workload in the sweep is additionally timed as the
reference harness does (moe/scripts/run_local.py:33: warmup 3, 100 iterations,
5 trials; the median trial mean is reported) and with per-stage hipEvents on
the launch stream.  Expert weights rotate over 4 copies (5.6 GB) so that no
call finds its weights in the 256 MB MALL / L2 left by the previous one.

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
STAGE_MFMA_DTYPE = {"gemm1_swiglu": "fp8", "gemm2": "bf16"}
GPU_WORKLOADS = ("decode_t1", "decode_t1_s3", "small_t64", "prefill_t1024", "skewed_t8192")
DEFAULT_WORKLOAD = "skewed_t8192"
WEIGHT_COPIES = 4


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def stage_work(stage, T, n_sel, a_act):
    """(algorithmic bytes, flops, peak FLOP/s) of one launch of a stage."""
    if stage == "gemm1_swiglu":
        return (a_act * G1_BYTES_PER_EXPERT + T * (H + 56 * 4) + n_sel * I * 2,
                n_sel * G1_FLOPS_PER_PAIR, PEAK["fp8"])
    if stage == "gemm2":
        return (a_act * G2_BYTES_PER_EXPERT + n_sel * I * 2 + n_sel * H * 4,
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

    def call(self, i, events=None):
        c = self.cfg
        self.pkg.run(*self.tok, *self.w[i % len(self.w)], c.local_expert_offset, c.routed_scaling_factor,
                     self.out, stage_events=events)

    def counts(self):
        ws = self.pkg.workspace(self.out.device, self.T)
        off = self.pkg.intermediates(ws, self.T).expert_off.cpu().tolist()
        n_sel = off[E_LOCAL]
        a_act = sum(1 for e in range(E_LOCAL) if off[e + 1] > off[e])
        return n_sel, a_act


def time_steps(torch, wl, steps, warmup):
    for i in range(warmup):
        wl.call(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        wl.call(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def harness_protocol(torch, wl, iters, trials, warmup):
    """hipEvent-timed trials on the launch stream; returns (median trial mean ms, all)."""
    s = torch.cuda.current_stream()
    for i in range(warmup):
        wl.call(i)
    means = []
    for _ in range(trials):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(s)
        for i in range(iters):
            wl.call(i)
        b.record(s)
        b.synchronize()
        means.append(a.elapsed_time(b) / iters)
    means.sort()
    return means[len(means) // 2], means


def stage_times(pkg, torch, wl, iters):
    """Mean device time per stage (ms), from events recorded by the library on
    the stream it launches on."""
    nst = len(STAGES) + 1
    pool = pkg._lib.EventPool(nst * iters)
    try:
        for i in range(iters):
            wl.call(i, events=pool.ptr(i * nst))
        torch.cuda.synchronize()
        tot = [0.0] * len(STAGES)
        for i in range(iters):
            for s in range(len(STAGES)):
                tot[s] += pool.elapsed_ms(i * nst + s, i * nst + s + 1)
        return {st: tot[k] / iters for k, st in enumerate(STAGES)}
    finally:
        pool.close()


def measure(pkg, torch, wl, iters, trials, warmup):
    med, trials_ms = harness_protocol(torch, wl, iters, trials, warmup)
    st = stage_times(pkg, torch, wl, min(iters, 50))
    n_sel, a_act = wl.counts()
    T = wl.T
    B = a_act * BYTES_PER_EXPERT + T * BYTES_PER_TOKEN + BYTES_BIAS
    F = n_sel * FLOPS_PER_PAIR
    sec = med * 1e-3
    layer = roofline(B, F, PEAK["fp8"], sec)
    dom = max(STAGES, key=lambda k: st[k])
    kb, kf, kp = stage_work(dom, T, n_sel, a_act)
    kern = roofline(kb, kf, kp, st[dom] * 1e-3)
    kern.update({"kernel": dom, "ms": st[dom], "algo_bytes": kb, "algo_flops": kf})
    return {
        "workload": wl.name, "T": T, "local_expert_offset": wl.cfg.local_expert_offset, "seed": wl.cfg.seed,
        "n_sel": n_sel, "a_act": a_act, "latency_us": med * 1e3,
        "trial_means_us": [round(x * 1e3, 3) for x in trials_ms],
        "tflops": F / sec / 1e12, "gbps": B / sec / 1e9,
        "bound": layer["bound"], "roofline_frac": layer["frac"],
        "stage_us": {k: round(v * 1e3, 3) for k, v in st.items()},
        "dominant": kern,
    }


def measured_traffic(workload, stage):
    """HBM bytes per launch of `stage` on `workload` from the committed rocprofv3
    counter summaries (profiles/*.txt lines 'TRAFFIC stage=S workload=W
    fetch_bytes=F write_bytes=B', already scaled by the copy calibration), or
    None when no summary covers it."""
    import glob

    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.txt"))):
        for line in open(path):
            if not line.startswith("TRAFFIC "):
                continue
            kv = dict(tok.split("=", 1) for tok in line.split()[1:] if "=" in tok)
            if kv.get("stage") == stage and kv.get("workload") == workload:
                return int(kv["fetch_bytes"]) + int(kv["write_bytes"])
    return None


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


def cpu_baseline(pkg, torch, wl, budget_tokens):
    """The oracle (plain-C restatement of full-agent-pipeline/references/moe.py,
    including its dequantise-all-32-experts step, moe.py:107-118) on the host
    cores, on two token prefixes of the workload; a linear fit in routed pairs
    extrapolates to the whole workload."""
    import numpy as np

    from oracle import oracle as orc

    orc.lib()
    cfg = wl.cfg
    w = wl.w[0]
    host_w = (w[0].view(torch.uint8).cpu().numpy(), w[1].cpu().numpy(), w[2].view(torch.uint8).cpu().numpy(),
              w[3].cpu().numpy())
    tok = wl.tok
    host_t = (tok[0].cpu().numpy(), tok[1].view(torch.int16).cpu().numpy().view(np.uint16),
              tok[2].view(torch.uint8).cpu().numpy(), tok[3].cpu().numpy())
    x = orc.Inputs(*host_t, *host_w, orc.Config(cfg.name, cfg.T, cfg.local_expert_offset, cfg.seed,
                                                 cfg.hot_experts, cfg.hot_add, cfg.routed_scaling_factor))
    ids, _ = orc.route(host_t[0], host_t[1], cfg.routed_scaling_factor)
    le = ids - cfg.local_expert_offset
    local = (le >= 0) & (le < E_LOCAL)
    pairs_total = int(local.sum())
    pts = []
    for n in (budget_tokens, 2 * budget_tokens):
        toks = np.arange(min(n, cfg.T), dtype=np.int32)
        t0 = time.perf_counter()
        orc.moe(x, tokens=toks, dequant_all=True)
        dt = time.perf_counter() - t0
        pts.append((int(local[toks].sum()), dt))
        log(f"[bench] cpu oracle: {len(toks)} tokens, {pts[-1][0]} pairs, {dt:.2f}s")
    (p1, t1), (p2, t2) = pts
    slope = (t2 - t1) / max(p2 - p1, 1)
    est = t1 + slope * (pairs_total - p1)
    return {
        "value": est * 1e6, "unit": "us", "cores": orc.lib().orc_num_threads(), "kind": "port",
        "sample": (f"oracle (C restatement of moe.py incl. dequantise-all-experts) on tokens [0,{budget_tokens}) "
                   f"and [0,{2 * budget_tokens}) of {cfg.name} ({p1} / {p2} routed pairs: {t1:.2f} s / {t2:.2f} s); "
                   f"linear fit in pairs extrapolated to all {pairs_total} pairs"),
    }


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
                    help="comma-separated workloads timed with the harness protocol ('' = none)")
    ap.add_argument("--iters", type=int, default=100)
    ap.add_argument("--trials", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--cpu-tokens", type=int, default=1024)
    ap.add_argument("--no-quant", action="store_true", help="skip the activation-quantiser measurement")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="also run a plain device copy of this size (for PMC byte calibration)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (the layer is one expert-parallel rank's "
              "shard; no collectives are implemented). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    pkg = importlib.import_module("mlsys-contest-syfi-fully-agent_amd")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    pkg._lib.moe_lib()  # fails loudly if the HIP library is not built
    cache = {}

    sweep = [s for s in args.sweep.split(",") if s]
    results = {}
    for name in sweep:
        wl = Workload(pkg, torch, name, dev, cache)
        log(f"[bench] {name}: T={wl.T}")
        results[name] = measure(pkg, torch, wl, args.iters, args.trials, args.warmup)
        r = results[name]
        log(f"[bench] {name}: {r['latency_us']:.1f} us, n_sel={r['n_sel']} a_act={r['a_act']} "
            f"{r['tflops']:.1f} TFLOP/s {r['gbps']:.0f} GB/s frac={r['roofline_frac']:.3f} stages={r['stage_us']}")

    head = Workload(pkg, torch, args.workload, dev, cache)
    ms = time_steps(torch, head, args.steps, args.warmup)
    log(f"[bench] headline {args.workload}: {ms * 1e3:.1f} us/step over {args.steps} steps")
    hm = results.get(args.workload) or measure(pkg, torch, head, args.iters, args.trials, args.warmup)

    if args.copy_calib_mib:
        copy_calibration(torch, dev, args.copy_calib_mib)
    quant = {}
    if not args.no_quant:
        for Tq in (1024, 8192):
            quant[f"t{Tq}"] = measure_quantizer(pkg, torch, dev, Tq)
            log(f"[bench] quantize_hidden T={Tq}: {quant[f't{Tq}']['latency_us']:.1f} us "
                f"{quant[f't{Tq}']['gbps']:.0f} GB/s")

    dom = hm["dominant"]
    roof = {"bound": dom["bound"], "achieved": round(dom["achieved"], 3), "peak": dom["peak"],
            "unit": dom["unit"], "frac": round(dom["frac"], 4),
            "traffic": measured_traffic(args.workload, dom["kernel"]),
            "kernel": dom["kernel"], "kernel_us": round(dom["ms"] * 1e3, 3)}
    cpu = None if args.no_cpu else cpu_baseline(pkg, torch, head, args.cpu_tokens)

    line = {
        "metric": "MoE layer latency (us) + FP8 TFLOPS / HBM GB/s as % roofline, T=1..8192",
        "value": round(ms * 1e3, 3), "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8", "dtype_detail": "e4m3 x e4m3 MFMA (GEMM1), bf16 MFMA (GEMM2), fp32 accumulate", "data": "synthetic (seeded generator)",
        "config": {"workload": args.workload, "T": head.T, "local_expert_offset": head.cfg.local_expert_offset,
                   "seed": head.cfg.seed, "hot_experts": list(head.cfg.hot_experts), "hot_bias_add": head.cfg.hot_add,
                   "n_sel": hm["n_sel"], "a_act": hm["a_act"], "parallelism": "single GPU (one EP rank)"},
        "tflops": round(hm["tflops"], 2), "gbps": round(hm["gbps"], 1), "layer_roofline_frac": round(hm["roofline_frac"], 4),
        "roofline": roof,
        "cpu_baseline": cpu,
        "upstream_quantizer": quant or None,
        "per_workload": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                         for k, v in results.items()},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
