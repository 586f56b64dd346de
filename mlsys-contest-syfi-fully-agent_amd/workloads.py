"""Reader for flashinfer-bench trace-set datasets (the contest's on-disk
format) restricted to this layer's definition.

A trace set is a directory tree (flashinfer-bench 0.1.2, the reference's
pinned harness, `full-agent-pipeline/uv.lock:318-320`; opened by
`TraceSet.from_path(...)` at `moe/scripts/run_local.py:36` and
`full-agent-pipeline/scripts/seed_ref_cache.py:49`):

    <root>/definitions/<op_type>/<definition>.json   the operator's schema
    <root>/workloads/<op_type>/<definition>.jsonl    one workload per line
    <root>/blob/...                                   safetensors payloads

The definition JSON names the axes (`{"type": "const", "value": v}` or
`{"type": "var"}`), the inputs and outputs (`{"shape": [axis names],
"dtype": "float8_e4m3fn" | ...}`, shape null for scalars) and carries the
PyTorch reference as text (`full-agent-pipeline/references/README.md:3-5`).
Each workload line holds `{"definition": name, "workload": {"uuid", "axes":
{var axis: size}, "inputs": {name: spec}}}`, where a spec is
`{"type": "safetensors", "path": <relative to root>, "tensor_key": k}`,
`{"type": "scalar", "value": v}` or `{"type": "random"}`
(`seed_ref_cache.py:77-81` loads the safetensors ones before generating the
rest).

flashinfer-bench itself is not installed here, so its `gen_inputs` random
generator is not reproduced: "random" inputs come from this package's seeded
GPU generator (`synth`, the distributions of the benchmark configurations),
seeded from the workload uuid.  Safetensors files are read with the
safetensors loader, which executes nothing from the file.  The reference
`reference` text in a definition is never executed.
"""
from __future__ import annotations

import json
import os
import zlib
from dataclasses import dataclass, field

import torch

from . import synth

DEFINITION_NAME = "moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048"
OP_TYPE = "moe"

# The contract of moe.py:29-40 in the definition's own vocabulary: constant
# axes, then the inputs in `run` order (shape as axis names; None = scalar).
CONST_AXES = {
    "num_experts": 256,
    "num_local_experts": 32,
    "hidden_size": 7168,
    "intermediate_size": 2048,
    "gemm1_out_size": 4096,
    "num_hidden_blocks": 56,
    "num_intermediate_blocks": 16,
    "num_gemm1_out_blocks": 32,
}
VAR_AXES = ("seq_len",)
INPUTS = (
    ("routing_logits", ("seq_len", "num_experts"), "float32"),
    ("routing_bias", ("num_experts",), "bfloat16"),
    ("hidden_states", ("seq_len", "hidden_size"), "float8_e4m3fn"),
    ("hidden_states_scale", ("num_hidden_blocks", "seq_len"), "float32"),
    ("gemm1_weights", ("num_local_experts", "gemm1_out_size", "hidden_size"), "float8_e4m3fn"),
    ("gemm1_weights_scale", ("num_local_experts", "num_gemm1_out_blocks", "num_hidden_blocks"), "float32"),
    ("gemm2_weights", ("num_local_experts", "hidden_size", "intermediate_size"), "float8_e4m3fn"),
    ("gemm2_weights_scale", ("num_local_experts", "num_hidden_blocks", "num_intermediate_blocks"), "float32"),
    ("local_expert_offset", None, "int32"),
    ("routed_scaling_factor", None, "float32"),
)
OUTPUTS = (("output", ("seq_len", "hidden_size"), "bfloat16"),)

_DTYPES = {
    "float32": torch.float32,
    "float16": torch.float16,
    "bfloat16": torch.bfloat16,
    "float8_e4m3fn": torch.float8_e4m3fn,
    "int32": torch.int32,
    "int64": torch.int64,
}

# Scalars a workload may leave to the generator.
DEFAULT_SCALARS = {"local_expert_offset": 0, "routed_scaling_factor": 2.5}


class DatasetError(ValueError):
    """The dataset does not match this layer's definition or is malformed."""


@dataclass
class Definition:
    name: str
    op_type: str
    axes: dict
    inputs: dict
    outputs: dict
    raw: dict = field(repr=False, default_factory=dict)

    def shape(self, tensor: str, axes: dict) -> tuple | None:
        spec = self.inputs.get(tensor) or self.outputs[tensor]
        if spec.get("shape") is None:
            return None
        sizes = {k: v["value"] for k, v in self.axes.items() if v.get("type") == "const"}
        sizes.update(axes)
        return tuple(int(sizes[a]) for a in spec["shape"])


@dataclass
class Workload:
    uuid: str
    axes: dict
    inputs: dict

    @property
    def T(self) -> int:
        return int(self.axes["seq_len"])


def contract_definition() -> dict:
    """This layer's definition in the trace-set JSON schema (no reference
    text): what a dataset's definition file must agree with."""
    return {
        "name": DEFINITION_NAME,
        "op_type": OP_TYPE,
        "axes": {**{a: {"type": "var"} for a in VAR_AXES},
                 **{a: {"type": "const", "value": v} for a, v in CONST_AXES.items()}},
        "inputs": {n: {"shape": list(s) if s else None, "dtype": d} for n, s, d in INPUTS},
        "outputs": {n: {"shape": list(s), "dtype": d} for n, s, d in OUTPUTS},
    }


def parse_definition(obj: dict) -> Definition:
    """Check a definition object against the layer's contract (names, input
    order, shapes, dtypes, constant axes) and wrap it."""
    try:
        name, axes, ins, outs = obj["name"], obj["axes"], obj["inputs"], obj["outputs"]
    except KeyError as e:
        raise DatasetError(f"definition lacks field {e}") from None
    if name != DEFINITION_NAME:
        raise DatasetError(f"definition {name!r} is not {DEFINITION_NAME!r}")
    for a, v in CONST_AXES.items():
        got = axes.get(a, {})
        if got.get("type") != "const" or int(got.get("value", -1)) != v:
            raise DatasetError(f"axis {a!r}: expected const {v}, found {got}")
    for a in VAR_AXES:
        if axes.get(a, {}).get("type") != "var":
            raise DatasetError(f"axis {a!r} must be var")
    if list(ins) != [n for n, _, _ in INPUTS]:
        raise DatasetError(f"inputs {list(ins)} differ from run's parameters {[n for n, _, _ in INPUTS]}")
    for n, s, d in INPUTS:
        spec = ins[n]
        shape = spec.get("shape")
        if (tuple(shape) if shape else None) != s or spec.get("dtype") != d:
            raise DatasetError(f"input {n!r}: expected shape {s} dtype {d}, found {shape} {spec.get('dtype')}")
    for n, s, d in OUTPUTS:
        spec = outs.get(n)
        if spec is None or tuple(spec.get("shape") or ()) != s or spec.get("dtype") != d:
            raise DatasetError(f"output {n!r}: expected shape {s} dtype {d}, found {spec}")
    return Definition(name, obj.get("op_type", OP_TYPE), axes, ins, outs, obj)


def parse_workload(obj: dict) -> Workload:
    """One JSONL line (a trace holding only a workload) -> Workload."""
    if obj.get("definition") != DEFINITION_NAME:
        raise DatasetError(f"workload for {obj.get('definition')!r}, not {DEFINITION_NAME!r}")
    wl = obj.get("workload") or {}
    try:
        uuid, axes, ins = str(wl["uuid"]), dict(wl["axes"]), dict(wl["inputs"])
    except KeyError as e:
        raise DatasetError(f"workload lacks field {e}") from None
    if set(axes) != set(VAR_AXES) or int(axes["seq_len"]) < 0:
        raise DatasetError(f"workload {uuid}: axes {axes} must give seq_len >= 0 only")
    names = {n for n, _, _ in INPUTS}
    if set(ins) - names:
        raise DatasetError(f"workload {uuid}: unknown inputs {sorted(set(ins) - names)}")
    for n, spec in ins.items():
        kind = spec.get("type")
        if kind == "safetensors":
            if "path" not in spec or "tensor_key" not in spec:
                raise DatasetError(f"workload {uuid}: input {n!r} needs path and tensor_key")
        elif kind == "scalar":
            if "value" not in spec:
                raise DatasetError(f"workload {uuid}: scalar input {n!r} needs value")
        elif kind != "random":
            raise DatasetError(f"workload {uuid}: input {n!r} has unknown type {kind!r}")
    return Workload(uuid, axes, ins)


class TraceSet:
    """The layer's definition and workloads of one trace-set directory."""

    def __init__(self, root: str, definition: Definition, workloads: list[Workload]):
        self.root = root
        self.definition = definition
        self.workloads = workloads

    @classmethod
    def from_path(cls, root: str, definition: str = DEFINITION_NAME) -> "TraceSet":
        root = os.path.abspath(root)
        dpath = _find(root, "definitions", definition + ".json")
        wpath = _find(root, "workloads", definition + ".jsonl")
        with open(dpath) as f:
            defn = parse_definition(json.load(f))
        wls = []
        with open(wpath) as f:
            for ln, line in enumerate(f, 1):
                line = line.strip()
                if not line:
                    continue
                try:
                    obj = json.loads(line)
                except json.JSONDecodeError as e:
                    raise DatasetError(f"{wpath}:{ln}: {e}") from None
                wls.append(parse_workload(obj))
        return cls(root, defn, wls)

    def workload(self, uuid_prefix: str) -> Workload:
        hits = [w for w in self.workloads if w.uuid.startswith(uuid_prefix)]
        if len(hits) != 1:
            raise KeyError(f"{len(hits)} workloads match {uuid_prefix!r}")
        return hits[0]


def _find(root: str, kind: str, fname: str) -> str:
    base = os.path.join(root, kind)
    direct = os.path.join(base, OP_TYPE, fname)
    if os.path.isfile(direct):
        return direct
    for d, _, files in os.walk(base):
        if fname in files:
            return os.path.join(d, fname)
    raise DatasetError(f"{fname} not found under {base}")


def workload_seed(wl: Workload) -> int:
    """Seed of the generator for a workload's "random" inputs."""
    return zlib.crc32(wl.uuid.encode()) & 0x7FFFFFFF


def read_input(ts: TraceSet, wl: Workload, name: str):
    """A workload's stored value of one input: a CPU tensor (safetensors,
    checked against the definition's shape and dtype), a Python scalar
    ("scalar", or a one-element safetensors entry for a scalar input), or
    None when the workload leaves it to the generator ("random")."""
    from safetensors import safe_open

    spec = wl.inputs.get(name, {"type": "random"})
    dtype = ts.definition.inputs[name]["dtype"]
    if spec["type"] == "random":
        return None
    if spec["type"] == "scalar":
        return int(spec["value"]) if dtype.startswith("int") else float(spec["value"])
    path = os.path.normpath(os.path.join(ts.root, spec["path"]))
    if not path.startswith(ts.root + os.sep):
        raise DatasetError(f"{wl.uuid}: {name} path {spec['path']!r} leaves the dataset root")
    if not os.path.isfile(path):
        raise DatasetError(f"{wl.uuid}: {name}: {spec['path']} not found")
    with safe_open(path, framework="pt", device="cpu") as f:
        if spec["tensor_key"] not in f.keys():
            raise DatasetError(f"{wl.uuid}: {name}: no tensor {spec['tensor_key']!r} in {spec['path']}")
        t = f.get_tensor(spec["tensor_key"])
    want = ts.definition.shape(name, wl.axes)
    if want is None:
        if t.numel() != 1:
            raise DatasetError(f"{wl.uuid}: scalar {name} has {t.numel()} elements")
        v = t.reshape(()).item()
        return int(v) if dtype.startswith("int") else float(v)
    if tuple(t.shape) != want or t.dtype != _DTYPES[dtype]:
        raise DatasetError(f"{wl.uuid}: {name} is {tuple(t.shape)} {t.dtype}, definition says {want} {dtype}")
    return t.contiguous()


def load_inputs(ts: TraceSet, wl: Workload, device) -> list:
    """The ten arguments of `run` for one workload, in order: tensors on
    `device`, scalars as Python numbers.  "random" tensors come from the
    seeded GPU generator (a GPU device is then required); "random" scalars
    take the benchmark defaults (offset 0, routed scaling factor 2.5)."""
    device = torch.device(device)
    out = {}
    for name, _, _ in INPUTS:
        v = read_input(ts, wl, name)
        if v is not None:
            out[name] = v.to(device) if isinstance(v, torch.Tensor) else v
    missing = [n for n, s, _ in INPUTS if n not in out and s is not None]
    if missing:
        if device.type != "cuda":
            raise DatasetError(f"{wl.uuid}: random inputs {missing} need a GPU device (seeded GPU generator)")
        cfg = synth.Config(f"wl_{wl.uuid[:8]}", wl.T, 0, workload_seed(wl))
        gen = {}
        if any(not n.startswith("gemm") for n in missing):
            gen.update(zip([n for n, _, _ in INPUTS[:4]], synth.tokens(cfg, device)))
        if any(n.startswith("gemm") for n in missing):
            gen.update(zip([n for n, _, _ in INPUTS[4:8]], synth.weights(cfg.seed, device)))
        for n in missing:
            out[n] = gen[n]
    for n, d in DEFAULT_SCALARS.items():
        out.setdefault(n, d)
    return [out[n] for n, _, _ in INPUTS]


def allocate_output(wl: Workload, device) -> torch.Tensor:
    return torch.empty((wl.T, CONST_AXES["hidden_size"]), dtype=torch.bfloat16, device=device)


def write_synthetic_traceset(root: str, configs, device) -> "TraceSet":
    """A trace set of the benchmark configurations (`synth.CONFIGS` entries),
    for runs without the contest dataset: each workload stores its four
    token tensors (so routing, hot experts and the local window are exactly
    the configuration's) and its scalars, and leaves the weights "random"
    (seeded from the workload uuid)."""
    from safetensors.torch import save_file

    root = os.path.abspath(root)
    for sub in ("definitions", "workloads"):
        os.makedirs(os.path.join(root, sub, OP_TYPE), exist_ok=True)
    blob = os.path.join(root, "blob", "workloads", OP_TYPE, DEFINITION_NAME)
    os.makedirs(blob, exist_ok=True)
    with open(os.path.join(root, "definitions", OP_TYPE, DEFINITION_NAME + ".json"), "w") as f:
        json.dump(contract_definition(), f, indent=1)
    lines = []
    for cfg in configs:
        names = [n for n, _, _ in INPUTS[:4]]
        toks = {n: t.cpu().contiguous() for n, t in zip(names, synth.tokens(cfg, device))}
        rel = os.path.join("blob", "workloads", OP_TYPE, DEFINITION_NAME, f"{cfg.name}.safetensors")
        save_file(toks, os.path.join(root, rel))
        ins = {n: {"type": "safetensors", "path": rel, "tensor_key": n} for n in names}
        ins.update({n: {"type": "random"} for n, _, _ in INPUTS[4:8]})
        ins["local_expert_offset"] = {"type": "scalar", "value": cfg.local_expert_offset}
        ins["routed_scaling_factor"] = {"type": "scalar", "value": cfg.routed_scaling_factor}
        wl = {"uuid": f"synthetic-{cfg.name}", "axes": {"seq_len": cfg.T}, "inputs": ins}
        lines.append(json.dumps({"definition": DEFINITION_NAME, "solution": None, "evaluation": None,
                                 "workload": wl}))
    with open(os.path.join(root, "workloads", OP_TYPE, DEFINITION_NAME + ".jsonl"), "w") as f:
        f.write("\n".join(lines) + "\n")
    return TraceSet.from_path(root)
