"""Helpers shared by the GPU tests: GPU inputs, their host copies for the
oracle, and the tie-aware comparison of routing results."""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as orc

_weights_cache: dict = {}


def gpu_weights(pkg, seed, device):
    """(device tensors, host numpy copies) of the seed's expert weights."""
    key = (seed, str(device))
    if key not in _weights_cache:
        _weights_cache.clear()  # keep one seed resident at a time
        w = pkg.synth.weights(seed, device)
        host = (w[0].view(torch.uint8).cpu().numpy(), w[1].cpu().numpy(),
                w[2].view(torch.uint8).cpu().numpy(), w[3].cpu().numpy())
        _weights_cache[key] = (w, host)
    return _weights_cache[key]


def gpu_tokens(pkg, cfg, device, T=None):
    tok = pkg.synth.tokens(cfg, device, T)
    host = (tok[0].cpu().numpy(), tok[1].view(torch.int16).cpu().numpy().view(np.uint16),
            tok[2].view(torch.uint8).cpu().numpy(), tok[3].cpu().numpy())
    return tok, host


def oracle_inputs(cfg, tok_host, w_host):
    return orc.Inputs(*tok_host, *w_host, orc.Config(cfg.name, tok_host[0].shape[0], cfg.local_expert_offset,
                                                        cfg.seed, cfg.hot_experts, cfg.hot_add,
                                                        cfg.routed_scaling_factor))


def near_tie_tokens(logits, bias, rsf=2.5, ulps=8):
    """Tokens whose selection boundary (4th vs 5th group score, or 8th vs 9th
    expert score among the kept groups) is within `ulps` fp32 ulps: there the
    routing choice may legitimately differ (exact ties are resolved by the
    reference's sort algorithm; 1-ulp score differences can swap them)."""
    ids, w, s, sb = orc.route(logits, bias, rsf, want_scores=True)
    T = logits.shape[0]
    g = sb.reshape(T, 8, 32)
    top2 = np.sort(g, axis=2)[:, :, -2:].sum(axis=2, dtype=np.float32)
    gs = np.sort(top2, axis=1)[:, ::-1]
    gap_g = gs[:, 3] - gs[:, 4]
    tol_g = ulps * np.spacing(np.abs(gs[:, 3]).astype(np.float32))
    kept = np.zeros((T, 256), bool)
    for t in range(T):
        sel_groups = np.argsort(-top2[t], kind="stable")[:4]
        for gi in sel_groups:
            kept[t, gi * 32:(gi + 1) * 32] = True
    cand = np.where(kept, sb, -np.inf)
    cs = np.sort(cand, axis=1)[:, ::-1]
    gap_e = cs[:, 7] - cs[:, 8]
    tol_e = ulps * np.spacing(np.abs(cs[:, 7]).astype(np.float32))
    return (gap_g <= tol_g) | (gap_e <= tol_e)


def bf16_close(got, ref, atol=1e-2, rtol=1e-2):
    """Element-wise |got - ref| <= atol + rtol * |ref| (the layer's tolerance)."""
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    bad = ~(np.abs(got - ref) <= atol + rtol * np.abs(ref))
    return bad
