"""The CPU restatement of the activation quantiser (the step before the
layer; the reference holds no quantiser, so its convention -- absmax/448 per
128 columns, e4m3 round-to-nearest-even saturating -- is this build's own,
shared with the input generator).  Pinned by properties that a wrong scale, a
dropped NaN guard or a wrong rounding would break, and against torch's own
fp32 -> float8_e4m3fn cast for every in-range value."""
import numpy as np
import pytest
import torch

H, B = 7168, 128


def _bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (torch's .to(bfloat16))."""
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _f32(u16: np.ndarray) -> np.ndarray:
    return (u16.astype(np.uint32) << 16).view(np.float32)


def _rows(T, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float32)
    x *= np.exp2(rng.integers(-20, 20, size=(T, H // B, 1))).astype(np.float32).repeat(B, axis=2).reshape(T, H)
    return _bf16(x)


def test_scale_is_block_absmax_over_448(orc):
    x = _rows(5)
    q, sc = orc.quantize_hidden(x)
    a = np.abs(_f32(x)).reshape(5, H // B, B).max(axis=2).T  # [56, T]
    np.testing.assert_array_equal(sc, (a / np.float32(448.0)).astype(np.float32))


def test_block_maximum_encodes_to_448(orc):
    x = _rows(3, seed=1)
    q, sc = orc.quantize_hidden(x)
    xf = _f32(x).reshape(3, H // B, B)
    idx = np.abs(xf).argmax(axis=2)
    qb = q.reshape(3, H // B, B)
    top = np.take_along_axis(qb, idx[..., None], axis=2)[..., 0]
    assert set(np.unique(top & 0x7F)) == {0x7E}          # +-448, the largest finite e4m3
    assert np.array_equal(top >> 7, (np.take_along_axis(xf, idx[..., None], axis=2)[..., 0] < 0))


def test_matches_torch_float8_cast_of_scaled_values(orc):
    """Each code is torch's RNE cast of x / scale (all |x / scale| <= 448)."""
    x = _rows(4, seed=2)
    q, sc = orc.quantize_hidden(x)
    xf = _f32(x).reshape(4, H // B, B)
    y = xf / sc.T[..., None]                               # fp32 true division, as the restatement
    ref = torch.from_numpy(y.reshape(4, H)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(q, ref)


def test_dequantised_error_is_at_most_half_an_e4m3_step(orc):
    x = _rows(2, seed=3)
    q, sc = orc.quantize_hidden(x)
    deq = orc.e4m3_to_f32(q).reshape(2, H // B, B)
    y = _f32(x).reshape(2, H // B, B) / sc.T[..., None]
    ay = np.abs(y)
    step = np.where(ay < 2.0 ** -6, 2.0 ** -9, np.exp2(np.floor(np.log2(np.maximum(ay, 2.0 ** -6))) - 3))
    assert np.all(np.abs(deq - y) <= step / 2 + 1e-12)


def test_zero_nan_and_inf_blocks(orc):
    x = np.zeros((1, H), dtype=np.float32)
    x[0, B:2 * B] = np.linspace(-3, 3, B, dtype=np.float32)
    x[0, B + 5] = np.nan                                   # NaN stays out of the absmax
    x[0, 2 * B + 7] = np.inf                               # inf makes the block scale inf
    x[0, 2 * B + 8] = 1.0
    q, sc = orc.quantize_hidden(_bf16(x))
    assert sc[0, 0] == 1.0 and np.all(q[0, :B] == 0)      # all-zero block
    assert sc[1, 0] == np.float32(3.0) / np.float32(448.0)
    assert q[0, B + 5] & 0x7F == 0x7F                     # NaN -> NaN code
    assert np.isinf(sc[2, 0])
    assert q[0, 2 * B + 7] & 0x7F == 0x7F                 # inf / inf = NaN
    assert q[0, 2 * B + 8] == 0                           # finite / inf = 0


@pytest.mark.parametrize("T", [1, 17])
def test_rows_are_independent(orc, T):
    x = _rows(T, seed=4)
    q, sc = orc.quantize_hidden(x)
    q1, sc1 = orc.quantize_hidden(x[-1:])
    np.testing.assert_array_equal(q[-1:], q1)
    np.testing.assert_array_equal(sc[:, -1:], sc1)


# ---- the GPU kernel's fast arithmetic, checked exhaustively on the CPU ------
# tests/support/quant_fastpath.c restates the kernel's fast quotient
# (q = x*r, q' = fma(fma(-s, q, x), r, q), sign from x) with the same single
# IEEE fp32 operations and compares its e4m3 code with the oracle's correctly
# rounded x / s for every bf16 pair |x| <= absmax.

def _fastpath_lib():
    import ctypes
    import os

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "support", "_build", "libquant_fastpath.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (run __graft_entry__.build())")
    L = ctypes.CDLL(path)
    L.quant_fastpath_mismatches.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int,
                                            ctypes.POINTER(ctypes.c_uint64)]
    L.quant_fastpath_mismatches.restype = ctypes.c_uint64
    return L


def _mismatches(L, lo, hi, variant):
    import ctypes

    pairs = ctypes.c_uint64(0)
    bad = L.quant_fastpath_mismatches(lo, hi, variant, ctypes.byref(pairs))
    return int(bad), int(pairs.value)


def test_fast_quotient_exhaustive():
    """Every block maximum the kernel's fast path accepts (0, or 2^-96 <= amax
    < inf; bf16 bits 0 and 0x0F80..0x7F7F) and every bf16 |x| <= amax."""
    L = _fastpath_lib()
    bad, pairs = _mismatches(L, 0x0F80, 0x7F80, 0)
    assert pairs > 1_000_000_000
    assert bad == 0
    assert _mismatches(L, 0, 1, 0) == (0, 2)  # amax = 0: x = +-0


def test_fast_quotient_check_has_teeth():
    """Planted mistakes fail the same check: no correction step, no sign fix,
    and tiny block maxima (< 2^-96, which the kernel sends to its exact path)."""
    L = _fastpath_lib()
    assert _mismatches(L, 0x3F00, 0x3F80, 1)[0] > 0   # y = x * r
    assert _mismatches(L, 0x3F00, 0x3F80, 2)[0] > 0   # -0 loses its sign
    assert _mismatches(L, 0x0400, 0x0F80, 0)[0] > 0   # below the fast path's range
