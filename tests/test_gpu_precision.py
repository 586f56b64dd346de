"""Layer output at large magnitudes, where the absolute tolerance no longer
hides the rounding of intermediates.

The contest's own workloads reach output magnitudes of ~5e5
(moe/solution/cuda/moe.cu:876-880), where an element passes atol = rtol =
1e-2 only with about 7 significant bits left after cancellation: bf16
intermediates (act, GEMM2 rows) then fail several percent of the elements.
The layer carries act as a bf16 (hi, lo) pair and the GEMM2 rows in fp32.
Outputs are scaled up through hidden_states_scale (the layer is linear in
it up to SwiGLU, so outputs grow about as its square) and checked against
the oracle with the verdict driver's check.  Two bars, both this project's
own (no harness rule pins a match ratio: the reference's runner checks with
rtol = 100, atol = 1e10, moe/scripts/run_local.py:33, and the 0.998 of
moe/solution/cuda/moe.cu:1802 is one variant's observed ratio, not a rule):
  * the match-ratio verdict at 0.998, the looser bar a caller may apply;
  * a regression floor per case close to the measured matched fraction
    (prefill routing, T = 128: x30 0.99996, 33 of 917,504 elements outside;
    x300 0.99926), so any change that loses precision fails here.
The second routing (four experts that every token selects, T = 1024) runs
the path that sums those experts inside GEMM2 (routing weights folded into
GEMM1's rows): x30 0.999902, x300 0.998722, against 0.999902 and 0.998716
for the same inputs with the experts combined separately.
The strict allclose verdict and its failure count are printed.  It cannot be
required: GEMM1 runs on the fp8 MFMA, whose block
sums carry ~2^-15 rms error (tests/test_gpu_mfma_precision.py), so at these
magnitudes a few elements in 10^5 that cancel to near zero exceed 1%.  The
torch fp32 restatement of the definition on the GPU (verdict.reference_layer,
fp32 GEMMs in another summation order) is printed as the floor of an
implementation without fp8 tensor-core arithmetic."""
import numpy as np
import pytest
import torch

from util import gpu_tokens, gpu_weights, oracle_inputs

pytestmark = pytest.mark.gpu

H = 7168


# This project's own match-ratio bar (0.998 is the ratio one reference
# variant recorded, moe/solution/cuda/moe.cu:1802; no harness rule pins it).
MATCH_RATIO_BAR = 0.998
# Regression floors: the measured matched fractions less a margin of a few
# elements in 10^5 (prefill routing x30 0.999964, x300 0.999259; every-token
# experts x30 0.999902, x300 0.998722).
MATCHED_FLOOR = {("prefill_t1024", 30.0): 0.99990, ("prefill_t1024", 300.0): 0.99900,
                 ("skewed_t8192", 30.0): 0.99985, ("skewed_t8192", 300.0): 0.99850}


@pytest.mark.parametrize("name,T,factor", [("prefill_t1024", 128, 30.0), ("prefill_t1024", 128, 300.0),
                                           ("skewed_t8192", 1024, 30.0), ("skewed_t8192", 1024, 300.0)])
def test_large_magnitude_output(pkg, orc, cuda_device, name, T, factor):
    cfg = pkg.synth.CONFIGS[name]
    w, w_host = gpu_weights(pkg, cfg.seed, cuda_device)
    tok, host = gpu_tokens(pkg, cfg, cuda_device, T)
    tok = (tok[0], tok[1], tok[2], (tok[3] * factor).contiguous())
    host = (host[0], host[1], host[2], (host[3] * np.float32(factor)).astype(np.float32))
    print(f"large-magnitude case {name} factor={factor} T={T}", flush=True)
    out = torch.empty((T, H), dtype=torch.bfloat16, device=cuda_device)
    pkg.run(*tok, *w, cfg.local_expert_offset, cfg.routed_scaling_factor, out)
    torch.cuda.synchronize()

    x = oracle_inputs(cfg, host, w_host)
    ref_bits = orc.moe(x)
    ref = torch.from_numpy(ref_bits.view(np.int16)).view(torch.bfloat16).to(cuda_device)
    v = pkg.verdict
    chk_all = v.check_output(out, ref)
    chk_ratio = v.check_output(out, ref, required_matched_ratio=MATCH_RATIO_BAR)
    floor = v.check_output(v.reference_layer(*tok, *w, cfg.local_expert_offset, cfg.routed_scaling_factor), ref)
    mag = ref.float().abs()
    n = out.numel()
    fails = int(round((1.0 - chk_all.matched_ratio) * n))
    print(f"  max|ref| {mag.max().item():.4g}, median|ref| {mag.median().item():.4g}; "
          f"layer: matched {chk_all.matched_ratio:.6f}, strict allclose {chk_all.status} "
          f"({fails} of {n} elements outside atol=rtol=1e-2), {chk_ratio.status} at {MATCH_RATIO_BAR}, "
          f"max|err| {chk_all.max_abs_err:.4g}; torch fp32 floor: matched {floor.matched_ratio:.6f} ({floor.status})")
    assert mag.max().item() > 10 * factor  # the scaling did reach large magnitudes
    assert chk_ratio.status == v.PASSED
    floor_ratio = MATCHED_FLOOR[(name, factor)]
    assert chk_all.matched_ratio >= floor_ratio, (chk_all.matched_ratio, floor_ratio)
