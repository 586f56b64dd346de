"""The oracle against the reference's own outputs (fixtures written by
tests/golden/make_golden.py from full-agent-pipeline/references/moe.py)."""
import numpy as np
import pytest

from conftest import load_golden


def _bf16_bits(orc, w):
    return np.array([orc.lib().orc_f32_to_bf16(float(v)) for v in w.ravel()], np.uint16).reshape(w.shape)


@pytest.mark.parametrize("batch", ["rand", "skew", "ties"])
def test_routing_matches_reference(orc, batch):
    """Expert choice and bf16(weight) of every token equal the reference's,
    including its resolution of exact ties (ties batch)."""
    g = load_golden("route_reveal.npz")
    if batch == "ties":
        logits = g["ties_logits"]
        bias = np.zeros(256, np.uint16)
    else:
        base = orc.CONFIGS["plumbing_t16" if batch == "rand" else "skewed_t8192"]
        logits, _, _, _ = orc.make_tokens(orc.CONFIGS["plumbing_t16"], int(g["T_rand"]))
        _, bias, _, _ = orc.make_tokens(base, 1)
    sel = g[f"{batch}_sel"]
    ids, w = orc.route(logits, bias)
    for t in range(logits.shape[0]):
        assert sorted(np.nonzero(sel[t])[0].tolist()) == ids[t].tolist(), f"token {t}"
    np.testing.assert_array_equal(np.take_along_axis(sel, ids.astype(np.int64), 1), _bf16_bits(orc, w))


@pytest.mark.parametrize("name", ["plumbing_t16", "small_t64", "prefill_t1024"])
def test_layer_matches_reference(orc, name):
    """bf16 output rows: equal to the reference's except for rounding flips from
    the fp32 matmul summation order (one bf16 ulp, or 1e-6 absolute where the
    sum cancels to nearly zero)."""
    g = load_golden(f"out_{name}.npz")
    x = orc.make_inputs(orc.CONFIGS[name])
    out = orc.moe(x, tokens=g["rows"])
    ref = g["out"]
    assert (out == ref).mean() > 0.998
    a, b = orc.bf16_to_f32(out), orc.bf16_to_f32(ref)
    ulp = np.abs(b) * 2.0 ** -7  # bf16 ulp bound at |ref|
    assert (np.abs(a - b) <= ulp + 1e-6).all(), "beyond rounding distance of the reference"
    # which tokens produce output at all (routing + local window)
    ids, _ = orc.route(x.logits, x.bias)
    le = ids - x.cfg.local_expert_offset
    nz = np.nonzero(((le >= 0) & (le < 32)).any(axis=1))[0]
    np.testing.assert_array_equal(nz, g["nonzero_rows"])
