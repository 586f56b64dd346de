"""Properties the mathematics fixes for the oracle (independent of the
golden fixtures): routing invariants, exact scaling laws, row independence."""
import numpy as np
import pytest


def test_routing_invariants(orc):
    logits, bias, _, _ = orc.make_tokens(orc.CONFIGS["prefill_t1024"])
    ids, w, s, sb = orc.route(logits, bias, 2.5, want_scores=True)
    T = logits.shape[0]
    # sigmoid closed form, scores = s + bias
    np.testing.assert_allclose(s, 1 / (1 + np.exp(-logits.astype(np.float64))), rtol=1e-6)
    np.testing.assert_array_equal(sb, s + orc.bf16_to_f32(bias)[None, :])
    g = sb.reshape(T, 8, 32)
    top2 = np.sort(g, axis=2)[:, :, -2:].sum(axis=2, dtype=np.float32)
    for t in range(T):
        assert len(set(ids[t])) == 8
        groups = np.argsort(-top2[t], kind="stable")[:4]
        assert set(ids[t] // 32) <= set(groups.tolist())
        kept = np.concatenate([np.arange(gi * 32, gi * 32 + 32) for gi in groups])
        best = kept[np.argsort(-sb[t, kept], kind="stable")[:8]]
        assert sorted(best.tolist()) == ids[t].tolist()
    # weights: un-biased sigmoid, normalised then scaled by rsf
    sel = np.take_along_axis(s, ids.astype(np.int64), 1)
    np.testing.assert_allclose(w, sel / sel.sum(1, keepdims=True) * 2.5, rtol=1e-6)
    np.testing.assert_allclose(w.sum(1), 2.5, rtol=1e-6)


def test_brute_force_tiny_routing(orc):
    """Hand-built scores: group 3 and 5 dominate, then 1 and 6."""
    logits = np.full((1, 256), -8.0, np.float32)
    for gi, v in ((3, 6.0), (5, 5.0), (1, 4.0), (6, 3.0)):
        logits[0, gi * 32:gi * 32 + 3] = [v, v - 0.5, v - 1.0]
    bias = np.zeros(256, np.uint16)
    ids, w = orc.route(logits, bias)
    expect = sorted([96, 97, 98, 160, 161, 162, 32, 33])
    assert ids[0].tolist() == expect


@pytest.fixture(scope="module")
def small(orc):
    cfg = orc.CONFIGS["small_t64"]
    return orc.make_inputs(cfg)


def test_rows_are_independent(orc, small):
    full = orc.moe(small)
    part = orc.moe(small, tokens=[5, 17, 40])
    np.testing.assert_array_equal(full[[5, 17, 40]], part)


def test_dequant_all_mode_same_bits(orc, small):
    a = orc.moe(small, tokens=np.arange(12))
    b = orc.moe(small, tokens=np.arange(12), dequant_all=True)
    np.testing.assert_array_equal(a, b)


def test_scaling_w2_by_two_doubles_output_exactly(orc, small):
    import dataclasses

    base = orc.moe(small, tokens=np.arange(16))
    x2 = dataclasses.replace(small, w2_scale=small.w2_scale * 2)
    dbl = orc.moe(x2, tokens=np.arange(16))
    np.testing.assert_array_equal(orc.bf16_to_f32(dbl), 2 * orc.bf16_to_f32(base))


def test_zero_down_weights_give_zero(orc, small):
    import dataclasses

    z = dataclasses.replace(small, w2=np.zeros_like(small.w2))
    assert not orc.moe(z, tokens=np.arange(8)).any()


def test_window_outside_experts_gives_zero(orc, small):
    assert not orc.moe(small, tokens=np.arange(8), local_expert_offset=256).any()
    assert not orc.moe(small, tokens=np.arange(8), local_expert_offset=-32).any()


def test_routed_scaling_is_linear(orc, small):
    a = orc.moe(small, tokens=np.arange(8), rsf=2.5)
    b = orc.moe(small, tokens=np.arange(8), rsf=5.0)
    np.testing.assert_array_equal(orc.bf16_to_f32(b), 2 * orc.bf16_to_f32(a))
