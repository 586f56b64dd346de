"""ctypes wrapper of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
and by bench.py's ``cpu_baseline`` leg, always as the checker or as the timed
CPU baseline, never as part of the product path.

The C sources restate ``full-agent-pipeline/references/moe.py`` (see
moe_oracle.c) and define the deterministic input generator (synth.c).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

H, I, E_LOCAL, E_GLOBAL, TOP_K, BLOCK = 7168, 2048, 32, 256, 8, 128
NH_BLK, NI_BLK, N2I_BLK = H // BLOCK, I // BLOCK, 2 * I // BLOCK

_DIR = os.path.dirname(os.path.abspath(__file__))
# MOE_ORACLE_LIB names another build of the same library (the tests' host-sanitized one)
_LIB_PATH = os.environ.get("MOE_ORACLE_LIB") or os.path.join(_DIR, "_build", "liboracle.so")
_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc). Returns the library path."""
    subprocess.run(["make", "-s", "-C", _DIR], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library not built: {_LIB_PATH} (run __graft_entry__.build())")
        L = ctypes.CDLL(_LIB_PATH)
        P, i64, u64, i32, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_int, ctypes.c_float
        L.orc_e4m3_to_f32.argtypes, L.orc_e4m3_to_f32.restype = [ctypes.c_uint8], f32
        L.orc_f32_to_e4m3.argtypes, L.orc_f32_to_e4m3.restype = [f32], ctypes.c_uint8
        L.orc_f32_to_bf16.argtypes, L.orc_f32_to_bf16.restype = [f32], ctypes.c_uint16
        L.orc_bf16_to_f32.argtypes, L.orc_bf16_to_f32.restype = [ctypes.c_uint16], f32
        L.orc_exp_f32.argtypes, L.orc_exp_f32.restype = [f32], f32
        L.synth_hash.argtypes, L.synth_hash.restype = [u64, ctypes.c_uint32, u64], u64
        L.synth_normal.argtypes, L.synth_normal.restype = [u64, ctypes.c_uint32, u64], f32
        L.synth_logits.argtypes = [u64, i64, P]
        L.synth_bias.argtypes = [u64, P, i32, f32, P]
        L.synth_hidden.argtypes = [u64, i64, P, P]
        L.synth_w13.argtypes = [u64, i32, i32, P, P]
        L.synth_w2.argtypes = [u64, i32, i32, P, P]
        L.orc_route.argtypes = [P, P, i64, f32, P, P, P, P]
        L.orc_quantize_hidden.argtypes = [P, i64, P, P]
        L.orc_moe.argtypes = [P, P, P, P, P, P, P, P, i64, f32, i64, P, i64, P, i32]
        L.orc_moe.restype = i32
        L.orc_expert_rows.argtypes = [P, P, i64, P, P, P, P, P, P, i64, P, P]
        L.orc_expert_rows.restype = i32
        L.orc_num_threads.restype = i32
        for fn in ("synth_logits", "synth_bias", "synth_hidden", "synth_w13", "synth_w2", "orc_route"):
            getattr(L, fn).restype = None
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---------------------------------------------------------------------------
# workload configurations (the benchmark's configs, stated in generator terms)
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class Config:
    name: str
    T: int
    local_expert_offset: int
    seed: int
    hot_experts: tuple = ()
    hot_add: float = 0.0
    routed_scaling_factor: float = 2.5


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


@dataclass
class Inputs:
    logits: np.ndarray
    bias: np.ndarray  # uint16 (bf16 bits)
    hs: np.ndarray  # uint8 (e4m3 bits)
    hs_scale: np.ndarray
    w13: np.ndarray | None
    w13_scale: np.ndarray | None
    w2: np.ndarray | None
    w2_scale: np.ndarray | None
    cfg: Config


def make_tokens(cfg: Config, T: int | None = None):
    T = cfg.T if T is None else T
    L = lib()
    logits = np.empty((T, E_GLOBAL), np.float32)
    L.synth_logits(cfg.seed, T, _p(logits))
    bias = np.empty(E_GLOBAL, np.uint16)
    hot = np.array(cfg.hot_experts, np.int32) if cfg.hot_experts else np.zeros(1, np.int32)
    L.synth_bias(cfg.seed, _p(hot), len(cfg.hot_experts), cfg.hot_add, _p(bias))
    hs = np.empty((T, H), np.uint8)
    hs_scale = np.empty((NH_BLK, T), np.float32)
    L.synth_hidden(cfg.seed, T, _p(hs), _p(hs_scale))
    return logits, bias, hs, hs_scale


def make_weights(seed: int, experts=(0, E_LOCAL)):
    """Full-size weight tensors; only experts in [e0, e1) are filled (rest zero)."""
    L = lib()
    e0, e1 = experts
    w13 = np.zeros((E_LOCAL, 2 * I, H), np.uint8)
    w13s = np.ones((E_LOCAL, N2I_BLK, NH_BLK), np.float32)
    w2 = np.zeros((E_LOCAL, H, I), np.uint8)
    w2s = np.ones((E_LOCAL, NH_BLK, NI_BLK), np.float32)
    L.synth_w13(seed, e0, e1, _p(w13), _p(w13s))
    L.synth_w2(seed, e0, e1, _p(w2), _p(w2s))
    return w13, w13s, w2, w2s


def make_inputs(cfg: Config, with_weights: bool = True, T: int | None = None) -> Inputs:
    logits, bias, hs, hs_scale = make_tokens(cfg, T)
    w = make_weights(cfg.seed) if with_weights else (None, None, None, None)
    return Inputs(logits, bias, hs, hs_scale, *w, cfg)


# ---------------------------------------------------------------------------
# oracle entry points
# ---------------------------------------------------------------------------
def route(logits: np.ndarray, bias: np.ndarray, rsf: float = 2.5, want_scores: bool = False):
    T = logits.shape[0]
    ids = np.empty((T, TOP_K), np.int32)
    w = np.empty((T, TOP_K), np.float32)
    s = np.empty((T, E_GLOBAL), np.float32) if want_scores else None
    sb = np.empty((T, E_GLOBAL), np.float32) if want_scores else None
    lib().orc_route(_p(np.ascontiguousarray(logits, np.float32)), _p(np.ascontiguousarray(bias)), T,
                    rsf, _p(ids), _p(w), _p(s), _p(sb))
    return (ids, w, s, sb) if want_scores else (ids, w)


def moe(x: Inputs, tokens=None, local_expert_offset=None, rsf=None, dequant_all=False) -> np.ndarray:
    """bf16 output rows (as uint16 bits) for `tokens` (default: all)."""
    T = x.logits.shape[0]
    off = x.cfg.local_expert_offset if local_expert_offset is None else local_expert_offset
    rsf = x.cfg.routed_scaling_factor if rsf is None else rsf
    tok = None if tokens is None else np.ascontiguousarray(tokens, np.int32)
    n = T if tok is None else len(tok)
    out = np.empty((n, H), np.uint16)
    rc = lib().orc_moe(_p(x.logits), _p(x.bias), _p(x.hs), _p(x.hs_scale), _p(x.w13), _p(x.w13_scale),
                       _p(x.w2), _p(x.w2_scale), off, rsf, T, _p(tok), n, _p(out), int(dequant_all))
    if rc != 0:
        raise MemoryError("orc_moe failed")
    return out


def expert_rows(x: Inputs, pair_token, pair_le, want_o=True):
    pt = np.ascontiguousarray(pair_token, np.int32)
    pl = np.ascontiguousarray(pair_le, np.int32)
    n = len(pt)
    c = np.empty((n, I), np.float32)
    o = np.empty((n, H), np.float32) if want_o else None
    rc = lib().orc_expert_rows(_p(x.hs), _p(x.hs_scale), x.hs.shape[0], _p(x.w13), _p(x.w13_scale),
                               _p(x.w2), _p(x.w2_scale), _p(pt), _p(pl), n, _p(c), _p(o))
    if rc != 0:
        raise MemoryError("orc_expert_rows failed")
    return c, o


def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    return (u16.astype(np.uint32) << 16).view(np.float32)


def e4m3_to_f32(u8: np.ndarray) -> np.ndarray:
    lut = np.array([lib().orc_e4m3_to_f32(i) for i in range(256)], np.float32)
    return lut[u8]


def quantize_hidden(x_bf16: np.ndarray):
    """bf16 bits [T, 7168] (uint16) -> (e4m3 bits uint8 [T, 7168], scales f32 [56, T])."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    T = x.shape[0]
    q = np.empty((T, H), dtype=np.uint8)
    sc = np.empty((H // 128, T), dtype=np.float32)
    lib().orc_quantize_hidden(_p(x), T, _p(q), _p(sc))
    return q, sc

