"""moe_fp8_ds_run_noalloc (no workspace argument, intermediates in the
library's static per-device scratch) against moe_fp8_ds_run, called through
the C ABI: bit-identical outputs on two calls in a row, the second with a
smaller T, plus the size limit."""
import ctypes

import numpy as np
import pytest
import torch

from util import gpu_tokens, gpu_weights

pytestmark = pytest.mark.gpu

H = 7168


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _call_run(pkg, tok, w, off, rsf, out):
    """moe_fp8_ds_run with a fresh workspace."""
    L = pkg._lib.moe_lib()
    T = tok[0].shape[0]
    ws = torch.empty(max(L.moe_fp8_ds_workspace_size(T), 256), dtype=torch.uint8, device=out.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = L.moe_fp8_ds_run(*[_p(t) for t in tok], *[_p(t) for t in w], off, rsf, _p(out), T, _p(ws),
                          ws.numel(), stream)
    assert rc == 0, pkg._lib.status_string(rc)


def _call_noalloc(pkg, tok, w, off, rsf, out):
    L = pkg._lib.moe_lib()
    T = tok[0].shape[0]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return L.moe_fp8_ds_run_noalloc(*[_p(t) for t in tok], *[_p(t) for t in w], off, rsf, _p(out), T, stream)


@pytest.mark.parametrize("name,T1,T2", [("small_t64", 64, 9), ("decode_t1_s3", 1, 1), ("plumbing_t16", 16, 3)])
def test_noalloc_matches_run(pkg, cuda_device, name, T1, T2):
    cfg = pkg.synth.CONFIGS[name]
    w, _ = gpu_weights(pkg, cfg.seed, cuda_device)
    for T in (T1, T2):  # the second call is smaller and reuses the scratch the first left behind
        tok, _ = gpu_tokens(pkg, cfg, cuda_device, T)
        print(f"noalloc case {name} T={T}", flush=True)
        ref = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=cuda_device)
        got = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=cuda_device)
        _call_run(pkg, tok, w, cfg.local_expert_offset, cfg.routed_scaling_factor, ref)
        rc = _call_noalloc(pkg, tok, w, cfg.local_expert_offset, cfg.routed_scaling_factor, got)
        assert rc == 0, pkg._lib.status_string(rc)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_noalloc_rejects_large_T(pkg, cuda_device):
    cfg = pkg.synth.CONFIGS["small_t64"]
    w, _ = gpu_weights(pkg, cfg.seed, cuda_device)
    T = pkg._lib.NOALLOC_MAX_TOKENS + 1
    tok, _ = gpu_tokens(pkg, cfg, cuda_device, T)
    out = torch.zeros((T, H), dtype=torch.bfloat16, device=cuda_device)
    assert _call_noalloc(pkg, tok, w, 0, 2.5, out) == pkg._lib.ERR_SCRATCH
    torch.cuda.synchronize()
    assert (out == 0).all()  # nothing was launched
    empty = [t[:0] for t in tok]
    assert _call_noalloc(pkg, empty, w, 0, 2.5, out[:0]) == 0


# Run in a fresh process: its first moe_fp8_ds_run_noalloc call (which looks
# up the device's scratch address) happens inside a graph capture.
_CAPTURE_SCRIPT = r"""
import ctypes, importlib, sys
import torch
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + "/tests")
from util import gpu_tokens, gpu_weights
pkg = importlib.import_module("mlsys-contest-syfi-fully-agent_amd")
dev = torch.device("cuda:0")
cfg = pkg.synth.CONFIGS["small_t64"]
w, _ = gpu_weights(pkg, cfg.seed, dev)
tok, _ = gpu_tokens(pkg, cfg, dev, 48)
T = 48
got = torch.full((T, 7168), float("nan"), dtype=torch.bfloat16, device=dev)
torch.cuda.synchronize()
# no kernel of the layer's library has run in this process before the capture
s = torch.cuda.Stream(device=dev)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=s):
    pkg.run_noalloc(*tok, *w, cfg.local_expert_offset, cfg.routed_scaling_factor, got)
torch.cuda.synchronize()
ref = torch.full((T, 7168), float("nan"), dtype=torch.bfloat16, device=dev)
pkg.run(*tok, *w, cfg.local_expert_offset, cfg.routed_scaling_factor, ref)
torch.cuda.synchronize()
other, _ = gpu_tokens(pkg, cfg, dev, 20)
other_out = torch.empty((20, 7168), dtype=torch.bfloat16, device=dev)
for rep in range(3):
    got.fill_(float("nan"))
    # eager work between replays: an eager no-alloc call that overwrites the
    # shared scratch with another input's intermediates
    pkg.run_noalloc(*other, *w, cfg.local_expert_offset, cfg.routed_scaling_factor, other_out)
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    ok = torch.equal(got.view(torch.int16), ref.view(torch.int16))
    print(f"noalloc captured first call: replay {rep} {'equal' if ok else 'DIFFERS'}", flush=True)
    if not ok:
        sys.exit(1)
print("noalloc capture ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture(cuda_device):
    """The first no-allocation call of a process, and its first call into the
    layer's library at all, is made inside a graph capture; every replay (with eager no-alloc calls on other inputs in
    between) equals moe_fp8_ds_run's bits."""
    import os
    import subprocess
    import sys

    from conftest import ROOT

    print("noalloc capture case: fresh process, T=48", flush=True)
    r = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT, ROOT], capture_output=True, text=True, timeout=110,
                       env=dict(os.environ))
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0 and "noalloc capture ok" in r.stdout
