"""gfx950 (MI355X) FP8 block-scale MoE layer
`moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048`.

The compute lives in HIP kernels behind the C ABI of include/moe_fp8_ds.h
(lib/libmoe_fp8_ds.so); `run` is the destination-passing entry point with the
contest solution's signature.  The directory name is not a Python identifier,
so import it with importlib:

    pkg = importlib.import_module("mlsys-contest-syfi-fully-agent_amd")
    pkg.run(...)
"""
from . import _lib, synth, verdict, workloads  # noqa: F401
from .moe import (intermediates, quantize_hidden, release_workspaces, route, run, run_noalloc,  # noqa: F401
                  workspace)

__all__ = ["run", "run_noalloc", "route", "intermediates", "workspace", "release_workspaces", "quantize_hidden", "synth",
           "workloads", "verdict"]
