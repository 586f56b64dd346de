"""The C ABI (include/*.h) without a GPU: the libraries load, export every
declared symbol, and reject bad arguments before launching anything."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADERS = {
    "moe_fp8_ds.h": "libmoe_fp8_ds.so",
    "moe_synth.h": "libmoe_synth.so",
}


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moe_\w+)\s*\(", text)))


@pytest.mark.parametrize("header,lib", sorted(HEADERS.items()))
def test_library_exports_every_declared_symbol(pkg, header, lib):
    so = ctypes.CDLL(os.path.join(pkg._lib.LIB_DIR, lib))
    names = declared(header)
    assert names, header
    missing = [n for n in names if not hasattr(so, n)]
    assert not missing, f"{lib} lacks {missing}"


def test_version_and_status_strings(pkg):
    L = pkg._lib.moe_lib()
    assert L.moe_fp8_ds_version() == 1
    for rc in (0, -1, -2, -3, -4, -5, -6, -7):
        assert pkg._lib.status_string(rc) != "unknown status"
    assert pkg._lib.status_string(-99) == "unknown status"


def test_layout_regions_disjoint_and_aligned(pkg):
    L = pkg._lib.moe_lib()
    for T in (0, 1, 3, 16, 1024, 8192, 14107):
        lay = pkg._lib.layout(T)
        assert lay.total == L.moe_fp8_ds_workspace_size(T)
        regions = sorted([
            (lay.block_hist, 128 * ((T + 3) // 4)), (lay.expert_off, 256), (lay.topk_ids, 32 * T), (lay.topk_w, 32 * T),
            (lay.pair_row, 32 * T), (lay.perm_token, 32 * T), (lay.perm_w, 32 * T), (lay.act, 8 * T * 2048 * 4),
            (lay.down, 8 * T * 7168 * 4 if T > 64 else 0)])
        for (a, na), (b, _) in zip(regions, regions[1:]):
            assert a % 256 == 0 and a + na <= b
        assert regions[-1][0] + regions[-1][1] <= lay.total
    assert L.moe_fp8_ds_workspace_size(-1) == 0
    assert L.moe_fp8_ds_workspace_size(L.moe_fp8_ds_max_tokens() + 1) == 0


def test_max_tokens_keeps_row_offsets_in_32_bits(pkg):
    """The wide GEMM1 addresses token rows of hidden_states with 32-bit byte
    offsets (token * 7168 + column): the largest accepted T keeps them exact."""
    L = pkg._lib.moe_lib()
    tmax = L.moe_fp8_ds_max_tokens()
    assert (tmax - 1) * 7168 + 7167 < 2 ** 32
    assert tmax >= 14107  # the contest dataset's largest T (moe.py:13)
    assert L.moe_fp8_ds_workspace_size(tmax) > 0


def test_python_thresholds_match_the_kernels(pkg):
    """The Python views' kernel thresholds are the ones the sources use."""
    csrc = os.path.join(ROOT, "mlsys-contest-syfi-fully-agent_amd", "csrc")
    common = open(os.path.join(csrc, "moe_common.hpp")).read()
    route = open(os.path.join(csrc, "route.hip")).read()
    assert re.search(r"constexpr int kGemm2StreamMaxTokens = (\d+);", common).group(1) == \
        str(pkg.moe.FUSED_COMBINE_MAX_TOKENS)
    assert re.search(r"constexpr int kRouteSingleMaxTokens = (\d+);", route).group(1) == \
        str(pkg.moe.ROUTE_ONE_WORKGROUP_MAX_TOKENS)


def test_noalloc_validation_without_gpu(pkg):
    """moe_fp8_ds_run_noalloc refuses T beyond its scratch before any HIP call."""
    L = pkg._lib.moe_lib()
    buf = ctypes.create_string_buffer(64 + 256)
    base = ctypes.addressof(buf)
    al = base + (-base) % 256  # never dereferenced
    p = al
    lim = pkg._lib.NOALLOC_MAX_TOKENS
    assert L.moe_fp8_ds_run_noalloc(p, p, p, p, p, p, p, p, 0, 2.5, p, lim + 1, None) == pkg._lib.ERR_SCRATCH
    assert L.moe_fp8_ds_run_noalloc(p, p, p, p, p, p, p, p, 0, 2.5, p, -1, None) == -2
    assert L.moe_fp8_ds_run_noalloc(p, p, p, p, p, p, p, p, 0, 2.5, p, 0, None) == 0
    # the same status as moe_fp8_ds_run for the same bad argument, checked in
    # the same order, before the scratch limit and the T == 0 no-op
    big = L.moe_fp8_ds_max_tokens() + 1
    assert L.moe_fp8_ds_run_noalloc(p, p, p, p, p, p, p, p, 0, 2.5, p, big, None) == -2
    assert _run(L, p, big, p, 1 << 40) == -2
    for rsf in (float("nan"), float("inf")):
        for T in (0, 4, lim + 1):
            assert L.moe_fp8_ds_run_noalloc(p, p, p, p, p, p, p, p, 0, rsf, p, T, None) == -6, (rsf, T)
            assert _run(L, p, T, p, 1 << 40, rsf=rsf) == -6, (rsf, T)
    # the header's limit is what the library enforces
    hdr = open(os.path.join(ROOT, "include", "moe_fp8_ds.h")).read()
    assert re.search(r"#define MOE_FP8_DS_NOALLOC_MAX_TOKENS (\d+)", hdr).group(1) == str(lim)


def _run(L, ptr, T, ws, ws_bytes, rsf=2.5, out=None):
    p = ptr
    return L.moe_fp8_ds_run(p, p, p, p, p, p, p, p, 0, rsf, p if out is None else out, T, ws, ws_bytes, None)


def test_argument_validation_without_gpu(pkg):
    """Every rejection happens on the host, before any HIP call."""
    L = pkg._lib.moe_lib()
    buf = ctypes.create_string_buffer(64 + 256)
    base = ctypes.addressof(buf)
    al = base + (-base) % 256  # 256-aligned fake address (never dereferenced)
    need = L.moe_fp8_ds_workspace_size(4)
    assert _run(L, al, 0, None, 0) == 0  # T == 0: no-op success
    assert _run(L, al, -1, al, need) == -2
    assert _run(L, al, L.moe_fp8_ds_max_tokens() + 1, al, 1 << 40) == -2
    assert _run(L, None, 4, al, need) == -1
    assert _run(L, al, 4, None, need) == -1
    assert _run(L, al, 4, al + 4, need) == -3
    assert _run(L, al + 8, 4, al, need) == -3
    assert _run(L, al, 4, al, need - 1) == -4
    assert _run(L, al, 4, al, need, rsf=float("nan")) == -6
    assert _run(L, al, 4, al, need, rsf=float("inf")) == -6
    assert L.moe_fp8_ds_route(None, al, 0, 2.5, 4, al, need, None) == -1
    assert L.moe_fp8_ds_route(al, al, 0, 2.5, 4, al, need - 256, None) == -4
    assert L.moe_fp8_ds_workspace_layout(4, None) == -1


def test_synth_validation_without_gpu(pkg):
    S = pkg._lib.synth_lib()
    assert S.moe_synth_logits(0, -1, None, None) == -2
    assert S.moe_synth_logits(0, 0, None, None) == 0
    assert S.moe_synth_hidden(0, 4, None, None, None) == -1
    assert S.moe_synth_w13(0, 0, 33, ctypes.c_void_p(16), ctypes.c_void_p(16), None) == -2
    assert S.moe_synth_bias(0, None, 9, 0.0, ctypes.c_void_p(16), None) == -1


def test_bench_probe_validation_without_gpu(pkg):
    """The roofline probes (lib/libmoe_bench.so) refuse what they cannot run
    before launching: an MFMA kind other than 0-3, a read size that the
    workgroups do not split evenly (hipErrorInvalidValue = 1)."""
    B = pkg._lib.bench_lib()
    assert B.moe_bench_mfma_loop(4, 1, 1, None, None) == 1
    assert B.moe_bench_mfma_loop(-1, 1, 1, None, None) == 1
    assert B.moe_bench_read_stream(None, 4096, None, 1, None) == 1
    assert B.moe_bench_read_stream(None, 1 << 20, None, 0, None) == 1


def test_python_entry_rejects_bad_shapes(pkg):
    import torch

    T = 2
    args = [torch.zeros(T, 256), torch.zeros(256, dtype=torch.bfloat16),
            torch.zeros(T, 7168, dtype=torch.float8_e4m3fn), torch.zeros(56, T),
            torch.zeros(1, dtype=torch.float8_e4m3fn), torch.zeros(1), torch.zeros(1, dtype=torch.float8_e4m3fn),
            torch.zeros(1)]
    with pytest.raises(AssertionError):
        pkg.run(*args, 0, 2.5, torch.zeros(T, 7168, dtype=torch.bfloat16))


def test_quantize_validation_without_gpu(pkg):
    L = pkg._lib.moe_lib()
    buf = ctypes.create_string_buffer(64 + 256)
    base = ctypes.addressof(buf)
    al = base + (-base) % 256  # never dereferenced: every case returns before a launch
    assert L.moe_fp8_ds_quantize_hidden(al, 0, al, al, None) == 0  # T == 0: no-op
    assert L.moe_fp8_ds_quantize_hidden(al, -1, al, al, None) == -2
    assert L.moe_fp8_ds_quantize_hidden(al, L.moe_fp8_ds_max_tokens() + 1, al, al, None) == -2
    assert L.moe_fp8_ds_quantize_hidden(None, 4, al, al, None) == -1
    assert L.moe_fp8_ds_quantize_hidden(al, 4, al, None, None) == -1
    assert L.moe_fp8_ds_quantize_hidden(al + 8, 4, al, al, None) == -3   # bf16 rows need 16 B
    assert L.moe_fp8_ds_quantize_hidden(al, 4, al + 8, al, None) == -3   # e4m3 rows need 16 B
    assert L.moe_fp8_ds_quantize_hidden(al, 4, al, al + 2, None) == -3   # scales need 4 B
