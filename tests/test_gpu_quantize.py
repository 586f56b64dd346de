"""GPU parity of the activation quantiser (moe_fp8_ds_quantize_hidden, the
step before the layer) against the CPU restatement, bit for bit, and its use
as the layer's input."""
import numpy as np
import pytest
import torch

from test_oracle_quantize import H, B, _bf16, _rows

pytestmark = pytest.mark.gpu


def _special_rows():
    x = np.zeros((3, H), dtype=np.float32)
    x[0, B:2 * B] = np.linspace(-3, 3, B, dtype=np.float32)
    x[0, B + 5] = np.nan
    x[0, 2 * B + 7] = np.inf
    x[0, 2 * B + 8] = -2.5
    x[1, :] = np.float32(3.0e38) * np.sign(np.sin(np.arange(H, dtype=np.float32)))
    x[2, :] = np.float32(1e-38) * np.cos(np.arange(H, dtype=np.float32))   # bf16 subnormal range
    x[2, 3] = -0.0
    return _bf16(x)


@pytest.mark.parametrize("T", [1, 15, 16, 17, 300, 2048, 2049])  # one row per workgroup up to 2048, four beyond
def test_quantize_matches_oracle(pkg, orc, cuda_device, T):
    host = _rows(T, seed=T)
    if T >= 3:
        host[:3] = _special_rows()
    q_ref, sc_ref = orc.quantize_hidden(host)
    x = torch.from_numpy(host.view(np.int16)).view(torch.bfloat16).to(cuda_device)
    print(f"quantize T={T}", flush=True)
    q, sc = pkg.quantize_hidden(x)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)
    np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), sc_ref.view(np.uint32))


def test_quantize_zero_tokens_is_noop(pkg, cuda_device):
    x = torch.empty((0, H), dtype=torch.bfloat16, device=cuda_device)
    q, sc = pkg.quantize_hidden(x)
    assert q.shape == (0, H) and sc.shape == (H // B, 0)


def test_quantized_rows_feed_the_layer(pkg, orc, cuda_device):
    """quantize -> run equals run on the restatement's quantised inputs."""
    from util import gpu_weights

    T = 16
    host = _rows(T, seed=7)
    q_ref, sc_ref = orc.quantize_hidden(host)
    w, _ = gpu_weights(pkg, 0, cuda_device)
    logits = torch.randn(T, 256, generator=torch.Generator().manual_seed(7)).to(cuda_device)
    bias = torch.zeros(256, dtype=torch.bfloat16, device=cuda_device)
    x = torch.from_numpy(host.view(np.int16)).view(torch.bfloat16).to(cuda_device)
    q, sc = pkg.quantize_hidden(x)
    out_a = torch.empty(T, H, dtype=torch.bfloat16, device=cuda_device)
    out_b = torch.empty_like(out_a)
    pkg.run(logits, bias, q, sc, *w, 0, 2.5, out_a)
    qb = torch.from_numpy(q_ref).view(torch.float8_e4m3fn).to(cuda_device)
    pkg.run(logits, bias, qb, torch.from_numpy(sc_ref).to(cuda_device), *w, 0, 2.5, out_b)
    torch.cuda.synchronize()
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16))


def test_fp8_convert_instruction_exhaustive(cuda_device):
    """The fast path's fp32 -> e4m3 instruction equals the exact path's
    software round-to-nearest-even for every fp32 with |y| < 464 (the fast
    path converts only |y| <= 448 * (1 + 2^-22)), and packs bytes as the
    kernel assumes; tests/support/cvt_check.hip runs all 2^32 patterns."""
    import ctypes
    import os

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "support", "_build", "libcvt_check.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (run __graft_entry__.build())")
    L = ctypes.CDLL(path)
    counts = (ctypes.c_ulonglong * 6)()
    print("cvt_check: 2^32 fp32 patterns", flush=True)
    assert L.cvt_check(counts) == 0
    assert counts[0] == 0 and counts[1] == 0, list(counts)
    assert counts[5] == 0, list(counts)


def _fast_and_exact_rows():
    """Rows that send some passes down each path: a NaN, an infinity or a
    tiny block maximum (< 2^-96) in one block of a pass makes the whole pass
    exact; neighbouring passes of the same row stay fast.  Blocks also hold
    random bf16 bit patterns below their maximum (all exponents, subnormals,
    signed zeros)."""
    rng = np.random.default_rng(11)
    T = 64
    bits = rng.integers(0, 0x10000, size=(T, H), dtype=np.uint32).astype(np.uint16)
    amax = rng.integers(0x0F80, 0x7F80, size=(T, H // B), dtype=np.uint32).astype(np.uint16)
    mag = bits & 0x7FFF
    mag = np.where(mag > np.repeat(amax, B, axis=1), mag % (np.repeat(amax, B, axis=1) + 1), mag).astype(np.uint16)
    x = (bits & 0x8000) | mag
    x[:, ::B] = amax  # each block's maximum, positive
    x[1, 3 * B + 9] = 0x7FC1                                   # NaN in pass 0
    x[2, 9 * B + 1] = 0xFF80                                   # -inf in pass 1
    x[3, 17 * B:18 * B] = (np.arange(B) % 0x0F00).astype(np.uint16)  # tiny block in pass 2
    x[4, 24 * B:25 * B] = 0                                    # zero block: fast path, s = 1
    x[5, :] = 0x8000                                           # all -0
    return x


def test_quantize_fast_and_exact_paths(pkg, orc, cuda_device):
    host = _fast_and_exact_rows()
    q_ref, sc_ref = orc.quantize_hidden(host)
    x = torch.from_numpy(host.view(np.int16)).view(torch.bfloat16).to(cuda_device)
    print("quantize fast/exact rows T=64", flush=True)
    q, sc = pkg.quantize_hidden(x)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)
    np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), sc_ref.view(np.uint32))
