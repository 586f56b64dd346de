"""The trace-set reader (workloads.py): the definition contract, the
workload JSONL schema and safetensors inputs, on hand-made datasets in the
flashinfer-bench layout.  The contest dataset itself is not available
offline, so these datasets are written by the tests."""
import copy
import json
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file


@pytest.fixture(scope="module")
def W(pkg):
    return pkg.workloads


def _write_dataset(root, W, workloads, definition=None):
    d = os.path.join(root, "definitions", "moe")
    w = os.path.join(root, "workloads", "moe")
    os.makedirs(d, exist_ok=True)
    os.makedirs(w, exist_ok=True)
    with open(os.path.join(d, W.DEFINITION_NAME + ".json"), "w") as f:
        json.dump(definition or {**W.contract_definition(), "reference": "# text only, never executed"}, f)
    with open(os.path.join(w, W.DEFINITION_NAME + ".jsonl"), "w") as f:
        for wl in workloads:
            f.write(json.dumps({"definition": W.DEFINITION_NAME, "solution": None, "evaluation": None,
                                "workload": wl}) + "\n")


def _tokens(T, seed):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, 256, generator=g)
    bias = (0.1 * torch.randn(256, generator=g)).to(torch.bfloat16)
    hs = torch.randn(T, 7168, generator=g).to(torch.float8_e4m3fn)
    hs_scale = torch.rand(56, T, generator=g) + 0.5
    return {"routing_logits": logits, "routing_bias": bias, "hidden_states": hs, "hidden_states_scale": hs_scale}


def _st_inputs(path, keys, scalars):
    ins = {k: {"type": "safetensors", "path": path, "tensor_key": k} for k in keys}
    ins.update({k: {"type": "scalar", "value": v} for k, v in scalars.items()})
    return ins


def test_contract_round_trip(W):
    d = W.parse_definition(W.contract_definition())
    assert d.name == W.DEFINITION_NAME
    assert d.shape("gemm1_weights", {"seq_len": 5}) == (32, 4096, 7168)
    assert d.shape("hidden_states_scale", {"seq_len": 5}) == (56, 5)
    assert d.shape("local_expert_offset", {"seq_len": 5}) is None
    assert d.shape("output", {"seq_len": 3}) == (3, 7168)


@pytest.mark.parametrize("mutate", [
    lambda d: d.update(name="moe_other"),
    lambda d: d["axes"]["hidden_size"].update(value=4096),
    lambda d: d["axes"].update(seq_len={"type": "const", "value": 16}),
    lambda d: d["inputs"]["hidden_states"].update(dtype="bfloat16"),
    lambda d: d["inputs"]["hidden_states_scale"].update(shape=["seq_len", "num_hidden_blocks"]),
    lambda d: d.update(inputs=dict(reversed(list(d["inputs"].items())))),
    lambda d: d["outputs"]["output"].update(dtype="float32"),
    lambda d: d.pop("axes"),
])
def test_definition_mismatch_is_rejected(W, mutate):
    d = copy.deepcopy(W.contract_definition())
    mutate(d)
    with pytest.raises(W.DatasetError):
        W.parse_definition(d)


@pytest.mark.parametrize("wl", [
    {"uuid": "a", "axes": {"seq_len": 4}, "inputs": {"bogus": {"type": "random"}}},
    {"uuid": "a", "axes": {"seq_len": 4}, "inputs": {"hidden_states": {"type": "file"}}},
    {"uuid": "a", "axes": {"seq_len": 4}, "inputs": {"hidden_states": {"type": "safetensors", "path": "x"}}},
    {"uuid": "a", "axes": {"seq_len": 4}, "inputs": {"local_expert_offset": {"type": "scalar"}}},
    {"uuid": "a", "axes": {"tokens": 4}, "inputs": {}},
    {"axes": {"seq_len": 4}, "inputs": {}},
])
def test_malformed_workload_is_rejected(W, wl):
    with pytest.raises(W.DatasetError):
        W.parse_workload({"definition": W.DEFINITION_NAME, "workload": wl})


def test_reads_safetensors_and_scalars(W, tmp_path):
    root = str(tmp_path)
    os.makedirs(os.path.join(root, "blob"))
    t5, t1 = _tokens(5, 1), _tokens(1, 2)
    save_file(t5, os.path.join(root, "blob", "w5.safetensors"))
    save_file({**t1, "off": torch.tensor([32], dtype=torch.int32)}, os.path.join(root, "blob", "w1.safetensors"))
    wls = [
        {"uuid": "5555-aaaa", "axes": {"seq_len": 5},
         "inputs": _st_inputs("./blob/w5.safetensors", t5, {"local_expert_offset": 64, "routed_scaling_factor": 1.5})},
        {"uuid": "1111-bbbb", "axes": {"seq_len": 1},
         "inputs": {**_st_inputs("blob/w1.safetensors", t1, {}),
                    "local_expert_offset": {"type": "safetensors", "path": "blob/w1.safetensors", "tensor_key": "off"},
                    "gemm1_weights": {"type": "random"}}},
    ]
    _write_dataset(root, W, wls)
    ts = W.TraceSet.from_path(root)
    assert [w.uuid for w in ts.workloads] == ["5555-aaaa", "1111-bbbb"]
    a = ts.workload("5555")
    for k, v in t5.items():
        got = W.read_input(ts, a, k)
        assert got.dtype == v.dtype and torch.equal(got.view(torch.uint8), v.view(torch.uint8)), k
    assert W.read_input(ts, a, "local_expert_offset") == 64
    assert W.read_input(ts, a, "routed_scaling_factor") == 1.5
    assert W.read_input(ts, a, "gemm2_weights") is None
    b = ts.workload("1111")
    assert W.read_input(ts, b, "local_expert_offset") == 32
    assert torch.equal(W.read_input(ts, b, "routing_logits"), t1["routing_logits"])
    # random tensors need the GPU generator: on the CPU the reader says so
    with pytest.raises(W.DatasetError, match="GPU"):
        W.load_inputs(ts, a, "cpu")


def test_stored_tensor_must_match_definition(W, tmp_path):
    root = str(tmp_path)
    os.makedirs(os.path.join(root, "blob"))
    t = _tokens(3, 0)
    bad = {**t, "hidden_states_scale": t["hidden_states_scale"].t().contiguous(),  # [T, 56]: not transposed
           "routing_bias": t["routing_bias"].float()}
    save_file(bad, os.path.join(root, "blob", "bad.safetensors"))
    wl = {"uuid": "c", "axes": {"seq_len": 3}, "inputs": _st_inputs("blob/bad.safetensors", t, {})}
    esc = {"uuid": "d", "axes": {"seq_len": 3},
           "inputs": {"routing_logits": {"type": "safetensors", "path": "../outside.safetensors", "tensor_key": "x"}}}
    miss = {"uuid": "e", "axes": {"seq_len": 3},
            "inputs": {"routing_logits": {"type": "safetensors", "path": "blob/bad.safetensors", "tensor_key": "nope"}}}
    _write_dataset(root, W, [wl, esc, miss])
    ts = W.TraceSet.from_path(root)
    with pytest.raises(W.DatasetError, match="hidden_states_scale"):
        W.read_input(ts, ts.workloads[0], "hidden_states_scale")
    with pytest.raises(W.DatasetError, match="routing_bias"):
        W.read_input(ts, ts.workloads[0], "routing_bias")
    assert W.read_input(ts, ts.workloads[0], "routing_logits").shape == (3, 256)
    with pytest.raises(W.DatasetError, match="leaves the dataset root"):
        W.read_input(ts, ts.workloads[1], "routing_logits")
    with pytest.raises(W.DatasetError, match="no tensor"):
        W.read_input(ts, ts.workloads[2], "routing_logits")


def test_dataset_layout_errors(W, tmp_path):
    with pytest.raises(W.DatasetError, match="not found"):
        W.TraceSet.from_path(str(tmp_path))
    _write_dataset(str(tmp_path), W, [])
    with open(os.path.join(str(tmp_path), "workloads", "moe", W.DEFINITION_NAME + ".jsonl"), "a") as f:
        f.write("{not json\n")
    with pytest.raises(W.DatasetError, match="jsonl:1"):
        W.TraceSet.from_path(str(tmp_path))


def test_workload_seed_is_stable(W):
    wl = W.Workload("0f3c2f9e-1234", {"seq_len": 1}, {})
    assert W.workload_seed(wl) == W.workload_seed(W.Workload("0f3c2f9e-1234", {"seq_len": 7}, {}))
    assert W.workload_seed(wl) != W.workload_seed(W.Workload("0f3c2f9e-1235", {"seq_len": 1}, {}))
    assert 0 <= W.workload_seed(wl) < 2 ** 31
