"""How exactly the two MFMA instructions of the layer's GEMMs sum their
products, against exact (float64) dot products of the same operands.

The result fixes the layer's precision budget at large output magnitudes:
  * v_mfma_f32_16x16x32_bf16 (GEMM2, activation hi and lo halves x e4m3 W2
    widened to bf16) accumulates to fp32 accuracy;
  * v_mfma_f32_16x16x128_f8f6f4 (GEMM1, one 128-wide scale block per
    instruction) does not: its block sum is off by up to ~2^-13 of the sum of
    |products| (rms ~2^-15), so GEMM1's rows carry ~1e-5 relative error that no
    fp32 scaling outside the instruction removes.  The reference's native-e4m3
    path has the same class of error (fp8 tensor-core MMAs promoted to fp32
    every 32 K, moe/solution/cuda/moe.cu:1749-1762)."""
import ctypes
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "support", "_build", "libmfma_precision.so")


def _tiles(kind, A, B):
    L = ctypes.CDLL(LIB)
    L.mfma_tiles.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    n = A.shape[0]
    D = np.empty((n, 16, 16), np.float32)
    assert L.mfma_tiles(kind, n, A.ctypes.data, B.ctypes.data, D.ctypes.data) == 0
    return D


def _e4m3_codes(x):
    """fp32 [.., 128] rows -> e4m3 codes, each row scaled to absmax 448 (the
    layer's 1 x 128 / 128 x 128 block quantisation)."""
    s = np.abs(x).max(axis=-1, keepdims=True) / 448.0
    q = torch.from_numpy((x / s).astype(np.float32)).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).numpy()


def _rel_err(D, exact, absum):
    return np.abs(D.astype(np.float64) - exact) / absum


def test_f8f6f4_block_sum_precision(cuda_device):
    rng = np.random.default_rng(0)
    n = 512
    A = _e4m3_codes(rng.standard_normal((n, 16, 128)))
    B = _e4m3_codes(rng.standard_normal((n, 16, 128)))
    print("mfma precision: f8f6f4 16x16x128, gaussian block-quantised operands", flush=True)
    D = _tiles(0, A, B)
    fa = torch.from_numpy(A).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    fb = torch.from_numpy(B).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    exact = np.einsum("tmk,tnk->tmn", fa, fb)
    absum = np.einsum("tmk,tnk->tmn", np.abs(fa), np.abs(fb))
    e = _rel_err(D, exact, absum)
    rel = np.abs(D - exact) / np.abs(exact).clip(1e-30)
    print(f"  err / sum|p|: max 2^{np.log2(e.max()):.1f}, rms 2^{np.log2(np.sqrt((e ** 2).mean())):.1f}; "
          f"err / |sum|: median 2^{np.log2(np.median(rel) + 1e-300):.1f}")
    assert e.max() < 2.0 ** -11      # the bound the layer's precision analysis uses
    # products are exact (8 significant bits): only the summation loses bits
    one = np.zeros_like(A)
    one[:, :, 0] = A[:, :, 0]
    D1 = _tiles(0, one, B)
    assert np.array_equal(D1, (fa[:, :, None, 0] * fb[:, None, :, 0]).astype(np.float32))


def test_bf16_chain_is_fp32_accurate(cuda_device):
    rng = np.random.default_rng(1)
    n = 512
    x = rng.standard_normal((n, 16, 128)).astype(np.float32)
    hi = torch.from_numpy(x).to(torch.bfloat16)
    lo = (torch.from_numpy(x) - hi.float()).to(torch.bfloat16)
    fb = torch.from_numpy(_e4m3_codes(rng.standard_normal((n, 16, 128)))).view(torch.float8_e4m3fn).float()
    Bb = fb.to(torch.bfloat16)  # e4m3 values are exact in bf16
    print("mfma precision: bf16 16x16x32 chained over 128 K", flush=True)
    for part in (hi, lo):
        D = _tiles(1, part.view(torch.int16).numpy(), Bb.view(torch.int16).numpy())
        fa = part.double().numpy()
        exact = np.einsum("tmk,tnk->tmn", fa, fb.double().numpy())
        absum = np.einsum("tmk,tnk->tmn", np.abs(fa), np.abs(fb.double().numpy()))
        e = _rel_err(D, exact, absum)
        print(f"  err / sum|p|: max 2^{np.log2(e.max()):.1f}, rms 2^{np.log2(np.sqrt((e ** 2).mean())):.1f}")
        assert e.max() < 2.0 ** -20      # fp32 accumulation


def test_bf16_convert_instruction_exhaustive(cuda_device):
    """v_cvt_pk_bf16_f32, which the SwiGLU epilogues use to split each fp32
    activation into its bf16 (hi, lo) pair, rounds every finite and infinite
    fp32 exactly like software round-to-nearest-even, keeps NaN a NaN, and
    puts element 0 in the low half (tests/support/cvt_check.hip)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "support", "_build", "libcvt_check.so")
    L = ctypes.CDLL(path)
    counts = (ctypes.c_ulonglong * 3)()
    print("bf16_check: 2^32 fp32 patterns", flush=True)
    assert L.bf16_check(counts) == 0
    assert list(counts) == [0, 0, 0], list(counts)
