"""The harness-equivalent verdict driver (verdict.py): its tolerance check,
its aggregation, and its torch restatement of the definition's reference,
which is pinned against the reference's own output rows (tests/golden) and
against the CPU oracle."""
import math

import numpy as np
import pytest
import torch

from conftest import load_golden


@pytest.fixture(scope="module")
def V(pkg):
    return pkg.verdict


def test_check_allclose_and_errors(V):
    ref = torch.tensor([[1.0, -2.0, 0.0, 100.0]], dtype=torch.bfloat16)
    c = V.check_output(ref.clone(), ref)
    assert (c.status, c.max_abs_err, c.max_rel_err, c.matched_ratio) == ("PASSED", 0.0, 0.0, 1.0)
    # |d| <= atol + rtol*|ref|: 100 -> tolerance 1.01; 101 is inside, 102 is not
    out = ref.clone()
    out[0, 3] = 101.0
    assert V.check_output(out, ref).status == "PASSED"
    out[0, 3] = 102.0
    c = V.check_output(out, ref)
    assert c.status == "INCORRECT_NUMERICAL" and c.max_abs_err == 2.0 and c.matched_ratio == 0.75
    assert math.isclose(c.max_rel_err, 0.02, rel_tol=1e-6)
    # the relative error of a zero reference uses the 1e-8 floor
    out = ref.clone()
    out[0, 2] = 0.005
    c = V.check_output(out, ref)
    assert c.status == "PASSED" and math.isclose(c.max_rel_err, 0.005 / 1e-8, rel_tol=1e-2)


def test_check_match_ratio_mode(V):
    ref = torch.zeros(10, 10, dtype=torch.bfloat16)
    out = ref.clone()
    out[0, 0] = 1.0
    assert V.check_output(out, ref).status == "INCORRECT_NUMERICAL"
    assert V.check_output(out, ref, required_matched_ratio=0.99).status == "PASSED"
    assert V.check_output(out, ref, required_matched_ratio=0.995).status == "INCORRECT_NUMERICAL"


def test_check_nonfinite_shape_dtype(V):
    ref = torch.ones(2, 3, dtype=torch.bfloat16)
    out = ref.clone()
    out[1, 1] = float("nan")
    c = V.check_output(out, ref, required_matched_ratio=0.5)
    assert c.matched_ratio == pytest.approx(5 / 6) and c.max_abs_err == float("inf")
    assert V.check_output(out, ref).status == "INCORRECT_NUMERICAL"
    assert V.check_output(torch.ones(3, 2, dtype=torch.bfloat16), ref).status == "INCORRECT_SHAPE"
    assert V.check_output(torch.ones(2, 3), ref).status == "INCORRECT_DTYPE"
    assert V.check_output(torch.ones(0, 3, dtype=torch.bfloat16), torch.ones(0, 3, dtype=torch.bfloat16)).status == "PASSED"


def test_aggregate(V):
    per = [{"status": "PASSED", "speedup": 2.0, "max_abs_err": 1e-3, "max_rel_err": 0.1},
           {"status": "PASSED", "speedup": 8.0, "max_abs_err": 4e-3, "max_rel_err": 0.2},
           {"status": "PASSED", "speedup": 5.0, "max_abs_err": 2e-3, "max_rel_err": 0.05}]
    a = V.aggregate(per)
    assert a["correct"] and a["num_passed"] == 3 and a["num_workloads"] == 3
    assert a["mean_speedup"] == 5.0 and a["median_speedup"] == 5.0 and a["min_speedup"] == 2.0
    assert a["max_abs_err"] == 4e-3 and a["max_rel_err"] == 0.2
    per.append({"status": "RUNTIME_ERROR"})
    a = V.aggregate(per)
    assert not a["correct"] and a["num_passed"] == 3 and a["median_speedup"] == 5.0
    assert not V.aggregate([])["correct"]


def _torch_inputs(orc, x):
    return (torch.from_numpy(x.logits), torch.from_numpy(x.bias.view(np.int16)).view(torch.bfloat16),
            torch.from_numpy(x.hs).view(torch.float8_e4m3fn), torch.from_numpy(x.hs_scale),
            torch.from_numpy(x.w13).view(torch.float8_e4m3fn), torch.from_numpy(x.w13_scale),
            torch.from_numpy(x.w2).view(torch.float8_e4m3fn), torch.from_numpy(x.w2_scale),
            x.cfg.local_expert_offset, x.cfg.routed_scaling_factor)


@pytest.mark.parametrize("name", ["plumbing_t16", "small_t64"])
def test_reference_restatement_matches_reference_rows(V, orc, name):
    """reference_layer on the CPU reproduces the rows the reference's own
    moe.py wrote (same torch build, same op order), bit for bit, and agrees
    with the C oracle to bf16 rounding."""
    g = load_golden(f"out_{name}.npz")
    x = orc.make_inputs(orc.CONFIGS[name])
    torch.set_num_threads(8)
    out = V.reference_layer(*_torch_inputs(orc, x))
    bits = out.view(torch.int16).numpy().view(np.uint16)
    rows = np.asarray(g["rows"])
    eq = (bits[rows] == g["out"]).mean()
    print(f"{name}: {eq:.6f} of reference bits equal")
    assert eq == 1.0
    ora = orc.moe(x)
    a, b = orc.bf16_to_f32(bits), orc.bf16_to_f32(ora)
    assert (np.abs(a - b) <= np.abs(b) * 2.0 ** -7 + 1e-6).all()
