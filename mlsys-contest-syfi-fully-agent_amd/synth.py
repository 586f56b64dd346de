"""Synthetic workload of the benchmark configurations, generated on the GPU
by libmoe_synth.so (include/moe_synth.h) straight into torch device tensors.

The byte stream depends only on (seed, tensor) and matches the CPU generator
the tests use, so a configuration is fully described by the fields of
`Config`.  Token rows are prefix-stable: the first T' rows for a given seed do
not depend on T.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib

H, I, E_LOCAL, E_GLOBAL, BLOCK = 7168, 2048, 32, 256, 128


@dataclass(frozen=True)
class Config:
    name: str
    T: int
    local_expert_offset: int
    seed: int
    hot_experts: tuple = ()
    hot_add: float = 0.0
    routed_scaling_factor: float = 2.5


# The five workloads of the benchmark (names say what each one is).
CONFIGS = {
    "plumbing_t16": Config("plumbing_t16", 16, 0, 0),
    "decode_t1": Config("decode_t1", 1, 0, 0),
    # seed 0's decode token routes to no local expert; seed 3 is the first
    # seed whose token picks local experts (2 of them)
    "decode_t1_s3": Config("decode_t1_s3", 1, 0, 3),
    "small_t64": Config("small_t64", 64, 32, 0),
    "prefill_t1024": Config("prefill_t1024", 1024, 0, 1),
    "skewed_t8192": Config("skewed_t8192", 8192, 0, 0, (0, 8, 16, 24), 2.0),
}


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _s(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ok(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed ({rc})")


def tokens(cfg: Config, device, T: int | None = None, seed: int | None = None):
    """routing_logits, routing_bias, hidden_states, hidden_states_scale."""
    T = cfg.T if T is None else T
    seed = cfg.seed if seed is None else seed
    L = _lib.synth_lib()
    logits = torch.empty((T, E_GLOBAL), dtype=torch.float32, device=device)
    bias = torch.empty((E_GLOBAL,), dtype=torch.bfloat16, device=device)
    hs = torch.empty((T, H), dtype=torch.float8_e4m3fn, device=device)
    hs_scale = torch.empty((H // BLOCK, T), dtype=torch.float32, device=device)
    hot = (ctypes.c_int32 * max(1, len(cfg.hot_experts)))(*cfg.hot_experts)
    _ok(L.moe_synth_logits(seed, T, _p(logits), _s(device)), "moe_synth_logits")
    _ok(L.moe_synth_bias(seed, ctypes.cast(hot, ctypes.c_void_p), len(cfg.hot_experts), cfg.hot_add, _p(bias),
                         _s(device)), "moe_synth_bias")
    _ok(L.moe_synth_hidden(seed, T, _p(hs), _p(hs_scale), _s(device)), "moe_synth_hidden")
    return logits, bias, hs, hs_scale


def weights(seed: int, device, experts=(0, E_LOCAL)):
    """gemm1_weights, gemm1_weights_scale, gemm2_weights, gemm2_weights_scale.
    Experts outside [e0, e1) are left zero (scales one)."""
    L = _lib.synth_lib()
    e0, e1 = experts
    full = (e0, e1) == (0, E_LOCAL)
    alloc = torch.empty if full else torch.zeros
    w13 = alloc((E_LOCAL, 2 * I, H), dtype=torch.float8_e4m3fn, device=device)
    w2 = alloc((E_LOCAL, H, I), dtype=torch.float8_e4m3fn, device=device)
    w13s = torch.ones((E_LOCAL, 2 * I // BLOCK, H // BLOCK), dtype=torch.float32, device=device)
    w2s = torch.ones((E_LOCAL, H // BLOCK, I // BLOCK), dtype=torch.float32, device=device)
    _ok(L.moe_synth_w13(seed, e0, e1, _p(w13), _p(w13s), _s(device)), "moe_synth_w13")
    _ok(L.moe_synth_w2(seed, e0, e1, _p(w2), _p(w2s), _s(device)), "moe_synth_w2")
    return w13, w13s, w2, w2s


def inputs(cfg: Config, device, T: int | None = None):
    return (*tokens(cfg, device, T), *weights(cfg.seed, device))
