"""ctypes bindings of the package's HIP libraries (built by build.py into lib/).

Loading fails loudly when a library is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(_DIR, "lib")
# MOE_FP8_DS_LIB names another build of the same library (the tests' host-sanitized one)
MOE_LIB = os.environ.get("MOE_FP8_DS_LIB") or os.path.join(LIB_DIR, "libmoe_fp8_ds.so")
SYNTH_LIB = os.path.join(LIB_DIR, "libmoe_synth.so")
BENCH_LIB = os.path.join(LIB_DIR, "libmoe_bench.so")

# moe_fp8_ds_status (include/moe_fp8_ds.h)
OK, ERR_NULL, ERR_SHAPE, ERR_ALIGN, ERR_WORKSPACE, ERR_HIP, ERR_ARG, ERR_SCRATCH = 0, -1, -2, -3, -4, -5, -6, -7
# MOE_FP8_DS_NOALLOC_MAX_TOKENS: largest T of moe_fp8_ds_run_noalloc
NOALLOC_MAX_TOKENS = 64


class Layout(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in
                ("topk_ids", "topk_w", "pair_row", "expert_off", "perm_token", "perm_w", "act", "down", "block_hist", "total")]


_moe = None
_synth = None


def _need(path: str) -> None:
    if not os.path.exists(path):
        raise RuntimeError(f"HIP library missing: {path}; build it with __graft_entry__.build() "
                           f"or python mlsys-contest-syfi-fully-agent_amd/build.py")


def moe_lib() -> ctypes.CDLL:
    global _moe
    if _moe is None:
        _need(MOE_LIB)
        import torch  # noqa: F401  (torch's HIP runtime first: one runtime per process)

        L = ctypes.CDLL(MOE_LIB)
        P, i64, sz, dbl = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t, ctypes.c_double
        L.moe_fp8_ds_version.restype = ctypes.c_int
        L.moe_fp8_ds_status_string.argtypes, L.moe_fp8_ds_status_string.restype = [ctypes.c_int], ctypes.c_char_p
        L.moe_fp8_ds_max_tokens.restype = i64
        L.moe_fp8_ds_workspace_size.argtypes, L.moe_fp8_ds_workspace_size.restype = [i64], sz
        L.moe_fp8_ds_workspace_layout.argtypes = [i64, ctypes.POINTER(Layout)]
        L.moe_fp8_ds_workspace_layout.restype = ctypes.c_int
        L.moe_fp8_ds_run.argtypes = [P, P, P, P, P, P, P, P, i64, dbl, P, i64, P, sz, P]
        L.moe_fp8_ds_run.restype = ctypes.c_int
        L.moe_fp8_ds_run_profiled.argtypes = [P, P, P, P, P, P, P, P, i64, dbl, P, i64, P, sz, P, P]
        L.moe_fp8_ds_run_profiled.restype = ctypes.c_int
        L.moe_fp8_ds_run_noalloc.argtypes = [P, P, P, P, P, P, P, P, i64, dbl, P, i64, P]
        L.moe_fp8_ds_run_noalloc.restype = ctypes.c_int
        L.moe_fp8_ds_route.argtypes = [P, P, i64, dbl, i64, P, sz, P]
        L.moe_fp8_ds_route.restype = ctypes.c_int
        L.moe_fp8_ds_quantize_hidden.argtypes = [P, i64, P, P, P]
        L.moe_fp8_ds_quantize_hidden.restype = ctypes.c_int
        _moe = L
    return _moe


def synth_lib() -> ctypes.CDLL:
    global _synth
    if _synth is None:
        _need(SYNTH_LIB)
        import torch  # noqa: F401

        L = ctypes.CDLL(SYNTH_LIB)
        P, i64, u64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_int
        L.moe_synth_logits.argtypes = [u64, i64, P, P]
        L.moe_synth_bias.argtypes = [u64, P, i32, ctypes.c_float, P, P]
        L.moe_synth_hidden.argtypes = [u64, i64, P, P, P]
        L.moe_synth_w13.argtypes = [u64, i32, i32, P, P, P]
        L.moe_synth_w2.argtypes = [u64, i32, i32, P, P, P]
        for f in ("moe_synth_logits", "moe_synth_bias", "moe_synth_hidden", "moe_synth_w13", "moe_synth_w2"):
            getattr(L, f).restype = ctypes.c_int
        _synth = L
    return _synth


_bench = None


def bench_lib() -> ctypes.CDLL:
    """Microbenchmarks for bench.py's measured peaks (csrc/peaks.hip)."""
    global _bench
    if _bench is None:
        _need(BENCH_LIB)
        import torch  # noqa: F401

        L = ctypes.CDLL(BENCH_LIB)
        P = ctypes.c_void_p
        L.moe_bench_read_stream.argtypes = [P, ctypes.c_size_t, P, ctypes.c_int, P]
        L.moe_bench_mfma_loop.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P]
        L.moe_bench_trace_mark.argtypes = [ctypes.c_int, P]
        L.moe_bench_read_stream.restype = L.moe_bench_mfma_loop.restype = L.moe_bench_trace_mark.restype = ctypes.c_int
        _bench = L
    return _bench


def status_string(rc: int) -> str:
    return moe_lib().moe_fp8_ds_status_string(rc).decode()


def layout(T: int) -> Layout:
    lay = Layout()
    rc = moe_lib().moe_fp8_ds_workspace_layout(T, ctypes.byref(lay))
    if rc != OK:
        raise ValueError(f"moe_fp8_ds_workspace_layout({T}): {status_string(rc)}")
    return lay


_hip = None


def hip_lib() -> ctypes.CDLL:
    """The HIP runtime torch already loaded (imported first so that this and
    the package's libraries bind to one runtime instance)."""
    global _hip
    if _hip is None:
        import torch  # noqa: F401  (loads torch's libamdhip64.so.7)

        L = ctypes.CDLL("libamdhip64.so.7")
        P = ctypes.c_void_p
        L.hipEventCreate.argtypes = [ctypes.POINTER(P)]
        L.hipEventDestroy.argtypes = [P]
        L.hipEventSynchronize.argtypes = [P]
        L.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), P, P]
        for f in ("hipEventCreate", "hipEventDestroy", "hipEventSynchronize", "hipEventElapsedTime"):
            getattr(L, f).restype = ctypes.c_int
        _hip = L
    return _hip


class EventPool:
    """`n` timing-enabled hipEvents (raw handles for the C ABI)."""

    def __init__(self, n: int):
        L = hip_lib()
        self.events = (ctypes.c_void_p * n)()
        for i in range(n):
            ev = ctypes.c_void_p()
            rc = L.hipEventCreate(ctypes.byref(ev))
            if rc != 0:
                raise RuntimeError(f"hipEventCreate failed ({rc})")
            self.events[i] = ev
        self.n = n

    def ptr(self, first: int = 0):
        """Address of events[first..] as a hipEvent_t* argument."""
        return ctypes.c_void_p(ctypes.addressof(self.events) + first * ctypes.sizeof(ctypes.c_void_p))

    def elapsed_ms(self, a: int, b: int) -> float:
        L = hip_lib()
        ms = ctypes.c_float()
        rc = L.hipEventSynchronize(self.events[b])
        if rc == 0:
            rc = L.hipEventElapsedTime(ctypes.byref(ms), self.events[a], self.events[b])
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def close(self):
        L = hip_lib()
        for i in range(self.n):
            if self.events[i]:
                L.hipEventDestroy(self.events[i])
                self.events[i] = None
