"""Write the golden fixtures under tests/golden/ from the contest reference.

Run once, in the build container (the reference is not on the GPU box):

    python tests/golden/make_golden.py /root/reference/full-agent-pipeline/references/moe.py

It imports the reference `run` (full-agent-pipeline/references/moe.py:28-202)
and calls it on inputs from the oracle's deterministic generator.  Only data is
written (inputs are regenerated from their seeds by the tests; the fixtures hold
outputs plus the small hand-built inputs).

Fixtures
--------
route_reveal.npz
    The reference's expert choice and combination weights, read through its
    own `run`.  `run` returns only the layer output, so the weights are built to
    make that output reveal the routing: hidden = 1.0 everywhere; local expert
    le has gate row 0 and up row 2048 set to 1.0 over k < 128 (scales 1/128 and
    1/4, so G1[0] = 1 and G1[2048] = 32; silu(32) rounds to 32 in fp32, so
    C[0] = 32) and down row h = le set to 1.0 at i = 0 (scale 1/32, so
    O[le] = 1 exactly).  Hence
    output[t, le] = bf16(w[t, offset + le]) and every other column is 0.
    Eight calls (offset = 0, 32, ..., 224) cover all 256 experts.
    Three token batches: `rand` (seed-0 logits, seed-0 bias), `skew` (same
    logits, the skewed-prefill bias) and `ties` (logits from {-2..2}, zero bias:
    exact ties in every selection stage).
out_<name>.npz
    bf16 output rows of the real layer on generated configurations.
"""
from __future__ import annotations

import gc
import importlib.util
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as O  # noqa: E402

OUT_DIR = os.path.dirname(os.path.abspath(__file__))
H, I, E_LOCAL, E_GLOBAL = O.H, O.I, O.E_LOCAL, O.E_GLOBAL


def load_reference(path):
    spec = importlib.util.spec_from_file_location("reference_moe", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.run


def t_fp8(a):
    return torch.from_numpy(a).view(torch.float8_e4m3fn)


def t_bf16(a):
    return torch.from_numpy(a).view(torch.bfloat16)


def call(run, logits, bias, hs, hs_scale, w13, w13s, w2, w2s, offset, rsf=2.5):
    out = run(torch.from_numpy(logits), t_bf16(bias), t_fp8(hs), torch.from_numpy(hs_scale), t_fp8(w13),
              torch.from_numpy(w13s), t_fp8(w2), torch.from_numpy(w2s), int(offset), float(rsf))
    res = out.view(torch.int16).numpy().view(np.uint16).copy()
    del out
    gc.collect()
    return res


def reveal_weights():
    one = np.uint8(0x38)  # e4m3 1.0
    w13 = np.zeros((E_LOCAL, 2 * I, H), np.uint8)
    w13s = np.ones((E_LOCAL, O.N2I_BLK, O.NH_BLK), np.float32)
    w2 = np.zeros((E_LOCAL, H, I), np.uint8)
    w2s = np.ones((E_LOCAL, O.NH_BLK, O.NI_BLK), np.float32)
    for le in range(E_LOCAL):
        w13[le, 0, :128] = one
        w13[le, I, :128] = one
        w13s[le, 0, 0] = 1.0 / 128
        w13s[le, I // 128, 0] = 0.25
        w2[le, le, 0] = one
        w2s[le, le // 128, 0] = 1.0 / 32
    return w13, w13s, w2, w2s


def reveal(run, logits, bias, W):
    T = logits.shape[0]
    hs = np.full((T, H), 0x38, np.uint8)
    hs_scale = np.ones((O.NH_BLK, T), np.float32)
    sel = np.zeros((T, E_GLOBAL), np.uint16)
    for off in range(0, E_GLOBAL, E_LOCAL):
        t0 = time.time()
        out = call(run, logits, bias, hs, hs_scale, *W, off)
        assert not out[:, E_LOCAL:].any(), "reveal: unexpected nonzero column"
        sel[:, off:off + E_LOCAL] = out[:, :E_LOCAL]
        print(f"  reveal offset {off}: {time.time() - t0:.1f}s", flush=True)
    return sel  # bf16 bits of the weight, 0 where not selected


def main():
    ref_path = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/full-agent-pipeline/references/moe.py"
    run = load_reference(ref_path)
    torch.set_num_threads(os.cpu_count() or 8)

    # ---- routing reveal -------------------------------------------------
    W = reveal_weights()
    base = O.CONFIGS["plumbing_t16"]
    skew = O.CONFIGS["skewed_t8192"]
    T_R = 256
    logits, bias, _, _ = O.make_tokens(base, T_R)
    _, bias_skew, _, _ = O.make_tokens(skew, 1)
    rng = np.random.default_rng(1234)
    tie_logits = rng.integers(-2, 3, size=(64, E_GLOBAL)).astype(np.float32)
    tie_logits[0] = 0.0  # fully tied token
    tie_logits[1] = (np.arange(E_GLOBAL) % 2).astype(np.float32)  # two tied levels
    zero_bias = np.zeros(E_GLOBAL, np.uint16)
    fx = {}
    print("reveal rand", flush=True)
    fx["rand_sel"] = reveal(run, logits, bias, W)
    print("reveal skew", flush=True)
    fx["skew_sel"] = reveal(run, logits, bias_skew, W)
    print("reveal ties", flush=True)
    fx["ties_sel"] = reveal(run, tie_logits, zero_bias, W)
    fx["ties_logits"] = tie_logits
    fx["T_rand"] = np.int64(T_R)
    del W
    gc.collect()
    np.savez_compressed(os.path.join(OUT_DIR, "route_reveal.npz"), **fx)

    # ---- real-layer outputs --------------------------------------------
    cases = [("plumbing_t16", None, 16), ("small_t64", None, 12), ("prefill_t1024", None, 8)]
    for name, _, max_rows in cases:
        cfg = O.CONFIGS[name]
        t0 = time.time()
        x = O.make_inputs(cfg)
        out = call(run, x.logits, x.bias, x.hs, x.hs_scale, x.w13, x.w13_scale, x.w2, x.w2_scale,
                   cfg.local_expert_offset, cfg.routed_scaling_factor)
        nz = np.nonzero(out.any(axis=1))[0]
        keep = nz[:max_rows]
        np.savez_compressed(os.path.join(OUT_DIR, f"out_{name}.npz"), rows=keep.astype(np.int32),
                            out=out[keep], nonzero_rows=nz.astype(np.int32), T=np.int64(cfg.T))
        print(f"out {name}: {len(nz)} nonzero rows, kept {len(keep)}, {time.time() - t0:.1f}s", flush=True)
        del x, out
        gc.collect()


if __name__ == "__main__":
    main()
