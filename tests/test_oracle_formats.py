"""Scalar formats of the oracle, pinned exhaustively against closed forms and
torch's own dtype conversions (the reference converts with torch:
moe.py:95,107,114 fp8 -> fp32 and moe.py:202 fp32 -> bf16)."""
import math

import numpy as np
import torch


def test_e4m3_decode_all_codes(orc):
    L = orc.lib()
    codes = np.arange(256, dtype=np.uint8)
    ours = np.array([L.orc_e4m3_to_f32(int(c)) for c in codes], np.float32)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(theirs)
    assert np.array_equal(np.isnan(ours), nan) and nan.sum() == 2  # 0x7F, 0xFF
    np.testing.assert_array_equal(ours[~nan], theirs[~nan])
    # closed form: sign * 2^(e-7) * (1 + m/8), subnormal m * 2^-9
    for c in range(256):
        s, e, m = c >> 7, (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            continue
        v = (m / 8) * 2.0 ** -6 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
        assert ours[c] == (-v if s else v)
    assert ours[0x7E] == 448.0


def test_e4m3_encode_matches_torch_rne(orc):
    L = orc.lib()
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.uniform(-448, 448, 20000),
        rng.normal(0, 1, 20000),
        rng.normal(0, 0.01, 5000),
        np.array([0.0, -0.0, 2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -10, 2.0 ** -6, 447.99, 448.0, -448.0, 1.0625,
                  1.1875, 0.01171875]),
    ]).astype(np.float32)
    # all halfway points between adjacent finite codes
    vals = np.sort(np.unique(np.abs(torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy())))
    vals = vals[np.isfinite(vals)]
    mids = ((vals[1:].astype(np.float64) + vals[:-1]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids])
    ours = np.array([L.orc_f32_to_e4m3(float(v)) for v in x], np.uint8)
    theirs = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(ours, theirs)


def test_e4m3_encode_saturates(orc):
    L = orc.lib()
    assert L.orc_f32_to_e4m3(449.0) == 0x7E
    assert L.orc_f32_to_e4m3(1e30) == 0x7E
    assert L.orc_f32_to_e4m3(-1e30) == 0xFE
    assert L.orc_f32_to_e4m3(float("inf")) == 0x7E
    assert L.orc_f32_to_e4m3(float("nan")) & 0x7F == 0x7F


def test_bf16_rne_matches_torch(orc):
    L = orc.lib()
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2 ** 32, 50000, dtype=np.uint64).astype(np.uint32)
    bits = np.concatenate([bits, np.array([0x3F808000, 0x3F818000, 0x7F7FFFFF, 0x00008000, 0x80018000], np.uint32)])
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    ours = np.array([L.orc_f32_to_bf16(float(v)) for v in x], np.uint16)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)


def test_exp_is_correctly_rounded_double(orc):
    L = orc.lib()
    for v in np.linspace(-30, 30, 2001, dtype=np.float32):
        assert L.orc_exp_f32(float(v)) == np.float32(math.exp(float(v)))
