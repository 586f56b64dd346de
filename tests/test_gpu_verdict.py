"""The verdict driver end to end on the GPU: a hand-made trace set (random,
safetensors and scalar inputs) through `run`, checked against the torch
restatement of the reference at the harness tolerance, timed, aggregated,
and through the script entry point."""
import json
import os

import pytest
import torch
from safetensors.torch import save_file

pytestmark = pytest.mark.gpu


def _dataset(root, W):
    os.makedirs(os.path.join(root, "definitions", "moe"))
    os.makedirs(os.path.join(root, "workloads", "moe"))
    os.makedirs(os.path.join(root, "blob"))
    with open(os.path.join(root, "definitions", "moe", W.DEFINITION_NAME + ".json"), "w") as f:
        json.dump(W.contract_definition(), f)
    g = torch.Generator().manual_seed(5)
    T = 16
    tok = {"routing_logits": torch.randn(T, 256, generator=g),
           "routing_bias": (0.1 * torch.randn(256, generator=g)).to(torch.bfloat16),
           "hidden_states": torch.randn(T, 7168, generator=g).to(torch.float8_e4m3fn),
           "hidden_states_scale": 0.01 * (torch.rand(56, T, generator=g) + 0.5)}
    save_file(tok, os.path.join(root, "blob", "t16.safetensors"))
    st = {k: {"type": "safetensors", "path": "blob/t16.safetensors", "tensor_key": k} for k in tok}
    wls = [
        {"uuid": "00000001-decode", "axes": {"seq_len": 1}, "inputs": {}},
        {"uuid": "00000016-stored", "axes": {"seq_len": 16},
         "inputs": {**st, "local_expert_offset": {"type": "scalar", "value": 32},
                    "routed_scaling_factor": {"type": "scalar", "value": 2.5}}},
        {"uuid": "00000064-random", "axes": {"seq_len": 64},
         "inputs": {"local_expert_offset": {"type": "scalar", "value": 0}}},
    ]
    with open(os.path.join(root, "workloads", "moe", W.DEFINITION_NAME + ".jsonl"), "w") as f:
        for wl in wls:
            f.write(json.dumps({"definition": W.DEFINITION_NAME, "workload": wl}) + "\n")
    return root


def test_verdicts_on_a_trace_set(pkg, cuda_device, tmp_path):
    W, V = pkg.workloads, pkg.verdict
    ts = W.TraceSet.from_path(_dataset(str(tmp_path), W))
    s = V.Settings(warmup=1, iterations=5, trials=2, ref_warmup=0, ref_iterations=1)
    print("verdict: 3 workloads", flush=True)
    rep = V.evaluate(pkg, ts, cuda_device, s, log=lambda m: print(m, flush=True))
    assert rep["correct"], rep
    assert rep["num_passed"] == 3
    for e in rep["per_workload"]:
        assert e["status"] == "PASSED" and e["max_abs_err"] < 1e-2
        assert e["latency_ms"] > 0 and e["speedup"] > 1.0
    # the stored tokens reached the layer: the stored workload's inputs are the file's
    args = W.load_inputs(ts, ts.workload("00000016"), cuda_device)
    assert args[8] == 32 and torch.equal(args[0].cpu(), W.read_input(ts, ts.workload("00000016"), "routing_logits"))


def test_planted_wrong_output_is_caught(pkg, cuda_device, tmp_path):
    """A layer output perturbed beyond tolerance on one element fails the
    check; within the match-ratio allowance it passes."""
    W, V = pkg.workloads, pkg.verdict
    ts = W.TraceSet.from_path(_dataset(str(tmp_path), W))
    wl = ts.workload("00000064")
    args = W.load_inputs(ts, wl, cuda_device)
    out = W.allocate_output(wl, cuda_device)
    pkg.run(*args, out)
    ref = V.reference_layer(*args)
    assert V.check_output(out, ref).status == "PASSED"
    flat = int(ref.float().abs().argmax())
    r, c = divmod(flat, ref.shape[1])
    assert abs(float(ref[r, c])) > 0.05
    out[r, c] = out[r, c] * 2
    assert V.check_output(out, ref).status == "INCORRECT_NUMERICAL"
    assert V.check_output(out, ref, required_matched_ratio=0.999).status == "PASSED"


def test_script_entry_point(pkg, cuda_device, tmp_path):
    V = pkg.verdict
    root = _dataset(str(tmp_path / "ds"), pkg.workloads)
    rep_path = str(tmp_path / "report.json")
    rc = V.main(["--dataset", root, "--limit", "2", "--warmup", "1", "--iterations", "3", "--trials", "1",
                 "--no-ref-timing", "--json", rep_path])
    assert rc == 0
    rep = json.load(open(rep_path))
    assert rep["num_workloads"] == 2 and rep["correct"]


def test_synthetic_traceset_reproduces_the_configuration(pkg, cuda_device, tmp_path):
    """--synthetic stores a benchmark configuration's token tensors: the
    reader hands back exactly what the generator makes for it."""
    cfg = pkg.synth.CONFIGS["small_t64"]
    ts = pkg.workloads.write_synthetic_traceset(str(tmp_path), [cfg], cuda_device)
    args = pkg.workloads.load_inputs(ts, ts.workloads[0], cuda_device)
    want = pkg.synth.tokens(cfg, cuda_device)
    for a, b in zip(args[:4], want):
        assert a.dtype == b.dtype and torch.equal(a.view(torch.uint8), b.view(torch.uint8))
    assert args[8] == 32 and args[9] == 2.5
    rc = pkg.verdict.main(["--synthetic", str(tmp_path / "s"), "--configs", "decode_t1_s3", "--warmup", "1",
                           "--iterations", "3", "--trials", "1", "--no-ref-timing"])
    assert rc == 0
