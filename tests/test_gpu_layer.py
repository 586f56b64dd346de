"""GPU parity of the whole layer (route -> GEMM1+SwiGLU -> GEMM2 -> combine)
against the CPU oracle and against the reference's own golden output rows,
through the C ABI (bf16 output within atol = rtol = 1e-2)."""
import numpy as np
import pytest
import torch

from conftest import load_golden
from util import bf16_close, gpu_tokens, gpu_weights, near_tie_tokens, oracle_inputs

pytestmark = pytest.mark.gpu

H, I = 7168, 2048


def run_layer(pkg, tok, w, off, rsf, fill=float("nan")):
    T = tok[0].shape[0]
    out = torch.full((T, H), fill, dtype=torch.bfloat16, device=tok[0].device)
    pkg.run(*tok, *w, off, rsf, out)
    torch.cuda.synchronize()
    return out


def sample_tokens(ids, off, n, rng, T):
    """Up to n tokens with at least one local expert, plus two without."""
    le = ids - off
    has = ((le >= 0) & (le < 32)).any(axis=1)
    loc = np.nonzero(has)[0]
    non = np.nonzero(~has)[0]
    pick = list(rng.choice(loc, size=min(n, loc.size), replace=False)) if loc.size else []
    pick += list(non[:2])
    return np.array(sorted(pick), np.int64)


# (config, local_expert_offset override, T override, tokens checked: None = every token)
LAYER_CASES = [
    ("plumbing_t16", None, None, None),
    ("decode_t1", None, None, None),
    ("decode_t1_s3", None, None, None),
    ("small_t64", None, None, None),
    ("prefill_t1024", None, None, None),
    ("skewed_t8192", None, None, None),
    ("small_t64", 224, None, None),
    ("small_t64", 240, 37, None),
    ("small_t64", -16, 21, None),
    ("prefill_t1024", 256, 128, None),
    # token counts on either side of each kernel-choice boundary
    ("small_t64", None, 17, None),        # first T past the in-GEMM1 routing
    # the hot experts take every token: experts of exactly 4 rows (act rows
    # spread over 4 loads per GEMM2 job), of 5 and 8 (8 loads) and of 9 (16)
    ("skewed_t8192", None, 4, None),
    ("skewed_t8192", None, 5, None),
    ("skewed_t8192", None, 8, None),
    ("skewed_t8192", None, 9, None),
    ("small_t64", None, 24, None),        # largest T of the one-workgroup routing launch
    ("small_t64", None, 25, None),        # routing plus a permutation launch
    # experts of more than 16 rows at T <= 64 (four hot experts of T rows):
    # the streaming GEMM1 launch runs the tiled kernel's tiles
    ("skewed_t8192", None, 17, None),
    ("skewed_t8192", None, 64, None),
    ("skewed_t8192", None, 40, None),
    ("prefill_t1024", None, 65, None),    # first T with the tiled GEMM1 and a combine pass
    # tiled GEMM1 tall tiles: two tall + one short tile of exactly 64 rows per
    # hot expert; prefill routing with tall and short tiles
    ("skewed_t8192", None, 320, None),
    ("prefill_t1024", None, 704, None),
    ("skewed_t8192", None, 1024, None),   # largest T of the tiled GEMM1 alone
    # 1025 <= T <= 1536: both GEMM1 kernels launched, the row counts choose one
    ("skewed_t8192", None, 1025, None),   # four hot experts: the wide kernel runs
    ("prefill_t1024", None, 1025, None),  # rows spread: the tiled kernel runs
    ("small_t64", None, 1536, None),      # the same at the range's top
    ("prefill_t1024", None, 1537, None),  # the wide kernel alone
    ("skewed_t8192", None, 2047, None),
    ("skewed_t8192", None, 2048, None),
    ("skewed_t8192", None, 4095, None),
    ("skewed_t8192", None, 4096, None),
    # the contest dataset's largest T (moe.py:13), every token
    ("skewed_t8192", None, 14107, None),
    # odd token counts on every kernel path, each with another routing window
    ("prefill_t1024", 96, 3, None),
    ("prefill_t1024", 160, 13, None),
    ("prefill_t1024", 64, 47, None),
    ("prefill_t1024", 192, 333, None),
    ("prefill_t1024", 128, 777, None),
    ("prefill_t1024", 32, 1537, None),
    ("prefill_t1024", 224, 3001, None),
    # windows that start inside a routing group (any offset is allowed)
    ("prefill_t1024", 77, 100, None),
    ("small_t64", 5, 64, None),
    ("skewed_t8192", 13, 2100, 384),
]


@pytest.mark.parametrize("name,offset,T,n_check", LAYER_CASES)
def test_layer_matches_oracle(pkg, orc, cuda_device, name, offset, T, n_check):
    cfg = pkg.synth.CONFIGS[name]
    off = cfg.local_expert_offset if offset is None else offset
    w, w_host = gpu_weights(pkg, cfg.seed, cuda_device)
    tok, host = gpu_tokens(pkg, cfg, cuda_device, T)
    print(f"layer case {name} offset={off} T={tok[0].shape[0]}", flush=True)
    check_layer(pkg, orc, cuda_device, cfg, off, tok, host, w, w_host, n_check)


# Other weights and tokens: generator seeds no config uses, each with another
# local window and a T on another kernel path (streaming, tiled with and
# without tall tiles, the two-kernel range, wide GEMM1).
SEED_CASES = [(5, 64, 50), (7, 160, 600), (9, 224, 1500), (11, 0, 800), (13, 96, 1100)]


@pytest.mark.parametrize("seed,offset,T", SEED_CASES)
def test_layer_seed_sweep(pkg, orc, cuda_device, seed, offset, T):
    cfg = pkg.synth.CONFIGS["prefill_t1024"]
    w, w_host = gpu_weights(pkg, seed, cuda_device)
    tok = pkg.synth.tokens(cfg, cuda_device, T, seed=seed)
    host = (tok[0].cpu().numpy(), tok[1].view(torch.int16).cpu().numpy().view(np.uint16),
            tok[2].view(torch.uint8).cpu().numpy(), tok[3].cpu().numpy())
    print(f"layer seed case seed={seed} offset={offset} T={T}", flush=True)
    check_layer(pkg, orc, cuda_device, cfg, offset, tok, host, w, w_host, None)


# A sweep over the tiled GEMM1's range and the two-kernel range (T = 65 to
# 1,536 in steps of 122): tile maps with and without tall tiles, every token.
SWEEP_CASES = [(name, T) for name in ("skewed_t8192", "prefill_t1024") for T in range(65, 1537, 122)]


@pytest.mark.parametrize("name,T", SWEEP_CASES)
def test_layer_sweep_mid_t(pkg, orc, cuda_device, name, T):
    cfg = pkg.synth.CONFIGS[name]
    w, w_host = gpu_weights(pkg, cfg.seed, cuda_device)
    tok, host = gpu_tokens(pkg, cfg, cuda_device, T)
    print(f"layer sweep case {name} T={T}", flush=True)
    check_layer(pkg, orc, cuda_device, cfg, cfg.local_expert_offset, tok, host, w, w_host, None)


# Routed scaling factors other than the configurations' 2.5 (the definition
# takes any value, moe.py:158): the factor passes through every routing
# implementation -- inside GEMM1 (T <= 16), the one-workgroup routing launch
# (T <= 24) and the routing kernel with its permutation launch -- and scales
# every output row, so a factor dropped or applied twice on any path fails.
RSF_CASES = [
    ("decode_t1_s3", 1.0, None),
    ("plumbing_t16", 0.37, None),
    ("small_t64", 7.0, 20),
    ("prefill_t1024", 1.0, 300),
    ("skewed_t8192", 0.125, 1500),
]


@pytest.mark.parametrize("name,rsf,T", RSF_CASES)
def test_layer_other_scaling_factors(pkg, orc, cuda_device, name, rsf, T):
    cfg = pkg.synth.CONFIGS[name]
    w, w_host = gpu_weights(pkg, cfg.seed, cuda_device)
    tok, host = gpu_tokens(pkg, cfg, cuda_device, T)
    print(f"layer rsf case {name} rsf={rsf} T={tok[0].shape[0]}", flush=True)
    check_layer(pkg, orc, cuda_device, cfg, cfg.local_expert_offset, tok, host, w, w_host, None, rsf=rsf)


# Every selection local (N_sel = 8 T, the largest row count the workspace
# holds): +10 on the bias of the 32 local experts puts their group first and
# all 8 picks in it, for every token, so the experts hold about T / 4 rows
# each -- experts of more than 16 rows in the streaming kernels at T = 64,
# tall tiles at T = 300, the two-kernel range (the wide tiles chosen) at
# T = 1100 and the wide GEMM1 alone at T = 3000.
ALL_LOCAL_CASES = [(1, None), (16, None), (64, None), (300, None), (1100, 256), (3000, 256)]


@pytest.mark.parametrize("T,n_check", ALL_LOCAL_CASES)
def test_layer_every_selection_local(pkg, orc, cuda_device, T, n_check):
    cfg = pkg.synth.CONFIGS["prefill_t1024"]
    off = cfg.local_expert_offset
    w, w_host = gpu_weights(pkg, cfg.seed, cuda_device)
    tok, host = gpu_tokens(pkg, cfg, cuda_device, T)
    bias = tok[1].float()
    bias[off:off + 32] += 10.0
    bias = bias.to(torch.bfloat16)
    tok = (tok[0], bias, tok[2], tok[3])
    host = (host[0], bias.view(torch.int16).cpu().numpy().view(np.uint16), host[2], host[3])
    ref_ids, _ = orc.route(host[0], host[1], cfg.routed_scaling_factor)
    assert ((ref_ids >= off) & (ref_ids < off + 32)).all(), "every pick local"
    print(f"layer every-selection-local case T={T}", flush=True)
    check_layer(pkg, orc, cuda_device, cfg, off, tok, host, w, w_host, n_check)
    if T > 16:  # the routing launches write the row offsets (at T <= 16 GEMM1 routes)
        offs = pkg.intermediates(pkg.workspace(cuda_device, T), T).expert_off.cpu().numpy()
        assert offs[32] == 8 * T and (np.diff(offs) >= 0).all()


# Experts that every token selects, summed inside GEMM2 (EVERY_TOKEN_FUSE_MIN_TOKENS):
# +10 on the bias of n local experts makes every token select them -- two
# (the fewest that are fused), eight (the most: every pick of every token),
# and with tokens ragged against the fused tiles' 64 rows.
FORCED_CASES = [(2, 1024, None), (8, 1024, 128), (2, 3000, 256), (8, 3001, 256), (3, 1025, 256)]


@pytest.mark.parametrize("n_forced,T,n_check", FORCED_CASES)
def test_layer_experts_of_every_token(pkg, orc, cuda_device, n_forced, T, n_check):
    cfg = pkg.synth.CONFIGS["prefill_t1024"]
    off = cfg.local_expert_offset
    w, w_host = gpu_weights(pkg, cfg.seed, cuda_device)
    tok, host = gpu_tokens(pkg, cfg, cuda_device, T)
    forced = off + np.arange(0, 32, 32 // n_forced)[:n_forced]
    bias = tok[1].float()
    bias[torch.as_tensor(forced, device=bias.device)] += 10.0
    bias = bias.to(torch.bfloat16)
    tok = (tok[0], bias, tok[2], tok[3])
    host = (host[0], bias.view(torch.int16).cpu().numpy().view(np.uint16), host[2], host[3])
    ref_ids, _ = orc.route(host[0], host[1], cfg.routed_scaling_factor)
    assert np.isin(forced, ref_ids).all() and all(np.isin(forced, row).all() for row in ref_ids[:64])
    print(f"layer forced-experts case n={n_forced} T={T}", flush=True)
    check_layer(pkg, orc, cuda_device, cfg, off, tok, host, w, w_host, n_check)
    offs = pkg.intermediates(pkg.workspace(cuda_device, T), T).expert_off.cpu().numpy()
    assert (np.diff(offs)[forced - off] == T).all()


def _random_cases(n, seed):
    """(routing config, T, window offset, token seed, weight seed, rsf) drawn
    from a fixed generator: T over every kernel path, any window start in
    [-31, 256), token seeds no configuration uses."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        name = ("prefill_t1024", "skewed_t8192", "small_t64")[int(rng.integers(3))]
        r = rng.random()
        T = int(rng.integers(1, 65)) if r < 0.35 else int(rng.integers(65, 1600)) if r < 0.8 else int(rng.integers(1600, 5000))
        out.append((name, T, int(rng.integers(-31, 256)), int(rng.integers(30, 60)),
                    None if rng.random() < 0.7 else int(rng.integers(30, 40)), float(rng.choice([2.5, 1.0, 0.5, 3.7]))))
    # grouped by weights, which the test helpers keep one seed of at a time
    return sorted(out, key=lambda c: (c[4] is None, c[4] or 0, c[0]))


@pytest.mark.parametrize("name,T,offset,seed,wseed,rsf", _random_cases(40, 2024))
def test_layer_random_cases(pkg, orc, cuda_device, name, T, offset, seed, wseed, rsf):
    cfg = pkg.synth.CONFIGS[name]
    w, w_host = gpu_weights(pkg, cfg.seed if wseed is None else wseed, cuda_device)
    tok = pkg.synth.tokens(cfg, cuda_device, T, seed=seed)
    host = (tok[0].cpu().numpy(), tok[1].view(torch.int16).cpu().numpy().view(np.uint16),
            tok[2].view(torch.uint8).cpu().numpy(), tok[3].cpu().numpy())
    print(f"layer random case {name} T={T} offset={offset} seed={seed} wseed={wseed} rsf={rsf}", flush=True)
    check_layer(pkg, orc, cuda_device, cfg, offset, tok, host, w, w_host, None if T <= 256 else 96, rsf=rsf)


def check_layer(pkg, orc, cuda_device, cfg, off, tok, host, w, w_host, n_check, rsf=None):
    """Every checked token whose routed expert ids equal the oracle's is
    compared element-wise; a token whose ids differ must be a near-tie of the
    fp32 scores (and is then left out)."""
    T = tok[0].shape[0]
    rsf = cfg.routed_scaling_factor if rsf is None else rsf
    out = run_layer(pkg, tok, w, off, rsf).float().cpu().numpy()
    assert np.isfinite(out).all(), "output not fully written / non-finite"
    gpu_ids = pkg.intermediates(pkg.workspace(cuda_device, T), T).topk_ids.cpu().numpy()

    ref_ids, _ = orc.route(host[0], host[1], rsf)
    tie = near_tie_tokens(host[0], host[1], rsf)
    differ = (np.sort(gpu_ids, axis=1) != ref_ids).any(axis=1)
    assert not (differ & ~tie).any(), f"ids differ outside near-ties: tokens {np.nonzero(differ & ~tie)[0][:8]}"
    rng = np.random.default_rng(T)
    toks = np.arange(T) if n_check is None or T <= n_check else sample_tokens(ref_ids, off, n_check, rng, T)
    toks = toks[~differ[toks]]
    x = oracle_inputs(cfg, host, w_host)
    ref = orc.bf16_to_f32(orc.moe(x, tokens=toks, local_expert_offset=off, rsf=rsf))
    got = out[toks]
    bad = bf16_close(got, ref)
    err = np.abs(got - ref)
    print(f"  near-tie tokens {int(tie.sum())} (ids differ on {int(differ.sum())}); checked {len(toks)} tokens: "
          f"max|err| {err.max() if err.size else 0:.3e}, max|ref| {np.abs(ref).max() if ref.size else 0:.3f}, "
          f"bit-equal {np.mean(got == ref) if ref.size else 1:.4f}")
    assert not bad.any(), f"{int(bad.sum())} elements outside tolerance, worst {err.max()}"
    # tokens without a local expert produce exact zeros
    le = ref_ids - off
    none = np.nonzero(~((le >= 0) & (le < 32)).any(axis=1))[0]
    assert (out[none] == 0).all()


@pytest.mark.parametrize("name", ["plumbing_t16", "small_t64", "prefill_t1024"])
def test_layer_matches_reference_golden(pkg, cuda_device, name):
    """Compare with bf16 rows written by the reference moe.py itself."""
    g = load_golden(f"out_{name}.npz")
    cfg = pkg.synth.CONFIGS[name]
    w, _ = gpu_weights(pkg, cfg.seed, cuda_device)
    tok, _ = gpu_tokens(pkg, cfg, cuda_device)
    out = run_layer(pkg, tok, w, cfg.local_expert_offset, cfg.routed_scaling_factor)
    got = out.float().cpu().numpy()
    ref = (g["out"].astype(np.uint32) << 16).view(np.float32)
    bad = bf16_close(got[g["rows"]], ref)
    assert not bad.any(), f"{int(bad.sum())} elements outside tolerance"
    nz = np.nonzero(np.abs(got).sum(axis=1) > 0)[0]
    np.testing.assert_array_equal(nz, g["nonzero_rows"])


INTERMEDIATE_CASES = [
    ("small_t64", None, None),          # row-streaming kernels
    ("skewed_t8192", 64, None),         # streaming GEMM1 launch with tiled tiles (experts of 64 rows)
    ("prefill_t1024", None, 200),
    ("skewed_t8192", 2304, 160),        # LDS-tiled / wide kernels, ragged last tiles
    # tiled GEMM2 with experts of a few to ~40 rows, every row: 16-row blocks
    # past a tile's rows are skipped per wave (0, 1 or 2 live blocks)
    ("prefill_t1024", 320, None),
    ("small_t64", 256, None),
    # tiled GEMM1 tile heights (64-row short tiles, 128-row tall tiles, chosen
    # per launch): the hot experts take every token, so T sets their rows.
    ("skewed_t8192", 128, None),        # tall map, experts of exactly 128 rows
    ("skewed_t8192", 129, None),        # short map, experts of 64 + 64 + 1 rows
    ("skewed_t8192", 193, None),        # tall map, a second tall tile of 65 rows
    ("skewed_t8192", 321, 400),         # tall map, three tall tiles, the last of 65 rows
    ("prefill_t1024", 704, 400),        # tall map, partly filled tall tiles among short ones
    # experts of every token summed inside GEMM2 (EVERY_TOKEN_FUSE_MIN_TOKENS):
    # weights folded in by the tiled GEMM1 (T = 1024) and the wide one (T =
    # 1100: the hot experts choose it), fused tiles with a ragged last row tile
    ("skewed_t8192", 1024, 300),
    ("skewed_t8192", 1100, 300),
]


@pytest.mark.parametrize("name,T,n_rows", INTERMEDIATE_CASES)
def test_intermediates_match_oracle(pkg, orc, cuda_device, name, T, n_rows):
    """SwiGLU activation rows (bf16 hi/lo pairs) and GEMM2 rows (fp32) per
    (token, expert) pair; with n_rows set, a sample that includes every expert's first and last
    row (tile edges)."""
    cfg = pkg.synth.CONFIGS[name]
    w, w_host = gpu_weights(pkg, cfg.seed, cuda_device)
    tok, host = gpu_tokens(pkg, cfg, cuda_device, T)
    T = tok[0].shape[0]
    print(f"intermediates case {name} T={T}", flush=True)
    run_layer(pkg, tok, w, cfg.local_expert_offset, cfg.routed_scaling_factor)
    r = pkg.intermediates(pkg.workspace(cuda_device, T), T)
    offs = r.expert_off.cpu().numpy()
    n = int(offs[32])
    perm = r.perm_token.cpu().numpy()[:n]
    le_all = np.searchsorted(offs, np.arange(n), side="right") - 1
    if n_rows is None or n <= n_rows:
        sel = np.arange(n)
    else:
        edges = np.concatenate([[offs[e], offs[e + 1] - 1] for e in range(32) if offs[e + 1] > offs[e]])
        rng = np.random.default_rng(n)
        sel = np.unique(np.concatenate([edges, rng.choice(n, n_rows, replace=False)]))
    act = pkg.moe.act_values(r.act[torch.as_tensor(sel, device=r.act.device)]).cpu().numpy()
    x = oracle_inputs(cfg, host, w_host)
    c_ref, o_ref = orc.expert_rows(x, perm[sel], le_all[sel])
    # Experts that every token selects (T rows each; at least two, from
    # EVERY_TOKEN_FUSE_MIN_TOKENS on):
    # their act rows carry the routing weight, and the first one's GEMM2 rows
    # hold each token's weighted sum over all of them (the others' rows are
    # not written).
    counts = np.diff(offs)
    fused = np.nonzero(counts == T)[0] if T >= pkg.moe.EVERY_TOKEN_FUSE_MIN_TOKENS else np.array([], np.int64)
    if fused.size < 2:
        fused = np.array([], np.int64)
    pw = r.perm_w.cpu().numpy()[:n]
    in_fused = np.isin(le_all[sel], fused)
    c_ref = np.where(in_fused[:, None], (c_ref * pw[sel][:, None]).astype(np.float32), c_ref)
    if fused.size:
        first = sel[le_all[sel] == fused[0]]  # rows of the first one: token = row - offs[first expert]
        toks = perm[first]
        o_sum = np.zeros((first.size, H), np.float64)
        for d in fused:
            rows_d = offs[d] + toks
            o_sum += orc.expert_rows(x, toks, np.full(toks.size, d))[1].astype(np.float64) * pw[rows_d][:, None]
        o_ref = o_ref.copy()
        o_ref[le_all[sel] == fused[0]] = o_sum.astype(np.float32)
        print(f"  experts of every token {fused.tolist()}: their rows checked as folded / summed")
    # act is carried as a bf16 (hi, lo) pair: fp32-level agreement (hi + lo is
    # within ~2^-17 of the fp32 value; the GEMM's fp32 summation order differs)
    ec = np.abs(act - c_ref)
    print(f"  act: max|err| {ec.max():.3e} (max|ref| {np.abs(c_ref).max():.3f}), "
          f"max rel {np.max(ec / (np.abs(c_ref) + 1e-3)):.3e}")
    bad_c = bf16_close(act, c_ref, atol=5e-4, rtol=1e-4)
    assert not bad_c.any(), f"act: {int(bad_c.sum())} bad, rows {np.unique(np.nonzero(bad_c)[0])[:8]}"
    if T <= pkg.moe.FUSED_COMBINE_MAX_TOKENS:
        assert r.down is None
        return  # GEMM2 rows are combined in registers, never stored
    down = r.down[torch.as_tensor(sel, device=r.down.device)].cpu().numpy()
    written = ~in_fused | (le_all[sel] == (fused[0] if fused.size else -1))
    down, o_ref = down[written], o_ref[written]
    eo = np.abs(down - o_ref)
    print(f"  down: max|err| {eo.max():.3e} (max|ref| {np.abs(o_ref).max():.3f})")
    bad_o = bf16_close(down, o_ref, atol=1e-4, rtol=1e-4)
    assert not bad_o.any(), f"down: {int(bad_o.sum())} bad, rows {np.unique(np.nonzero(bad_o)[0])[:8]}"


def test_zero_tokens_is_noop(pkg, cuda_device):
    cfg = pkg.synth.CONFIGS["plumbing_t16"]
    w, _ = gpu_weights(pkg, cfg.seed, cuda_device)
    tok, _ = gpu_tokens(pkg, cfg, cuda_device, 0)
    out = torch.empty((0, H), dtype=torch.bfloat16, device=cuda_device)
    pkg.run(*tok, *w, 0, 2.5, out)
    torch.cuda.synchronize()


def test_layer_deterministic(pkg, cuda_device):
    cfg = pkg.synth.CONFIGS["prefill_t1024"]
    w, _ = gpu_weights(pkg, cfg.seed, cuda_device)
    tok, _ = gpu_tokens(pkg, cfg, cuda_device)
    a = run_layer(pkg, tok, w, 0, 2.5)
    b = run_layer(pkg, tok, w, 0, 2.5, fill=0.0)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_workspace_needs_no_initialisation(pkg, cuda_device):
    """Garbage in the workspace does not change the result (no state is carried
    between calls)."""
    cfg = pkg.synth.CONFIGS["small_t64"]
    w, _ = gpu_weights(pkg, cfg.seed, cuda_device)
    tok, _ = gpu_tokens(pkg, cfg, cuda_device)
    ws = pkg.workspace(cuda_device, 64)
    outs = []
    for fill in (0x00, 0xAB, 0xFF):
        ws.fill_(fill)
        outs.append(run_layer(pkg, tok, w, cfg.local_expert_offset, cfg.routed_scaling_factor).view(torch.int16))
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


def test_concurrent_streams_use_their_own_workspaces(pkg, cuda_device):
    """Calls on two streams at once (different T, so each one's workspace
    holds different intermediates) give the bits of the same calls made one
    after the other, and each stream has its own workspace."""
    cfg = pkg.synth.CONFIGS["prefill_t1024"]
    w, _ = gpu_weights(pkg, cfg.seed, cuda_device)
    toks = [gpu_tokens(pkg, cfg, cuda_device, T)[0] for T in (300, 96)]
    want = [run_layer(pkg, tok, w, cfg.local_expert_offset, cfg.routed_scaling_factor) for tok in toks]
    streams = [torch.cuda.Stream(device=cuda_device) for _ in toks]
    outs = [torch.full((tok[0].shape[0], H), float("nan"), dtype=torch.bfloat16, device=cuda_device) for tok in toks]
    torch.cuda.synchronize()
    for _ in range(3):
        for s, tok, out in zip(streams, toks, outs):
            with torch.cuda.stream(s):
                pkg.run(*tok, *w, cfg.local_expert_offset, cfg.routed_scaling_factor, out)
    torch.cuda.synchronize()
    for got, ref in zip(outs, want):
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    ptrs = []
    for s, tok in zip(streams, toks):
        with torch.cuda.stream(s):
            ptrs.append(pkg.workspace(cuda_device, tok[0].shape[0]).data_ptr())
    assert ptrs[0] != ptrs[1]


def test_synth_matches_cpu_generator(pkg, orc, cuda_device):
    """The GPU generator writes the same bytes as the oracle's CPU generator."""
    for name in ("plumbing_t16", "skewed_t8192"):
        cfg = pkg.synth.CONFIGS[name]
        _, host = gpu_tokens(pkg, cfg, cuda_device, 64)
        ref = orc.make_tokens(orc.CONFIGS[name], 64)
        for a, b in zip(host, ref):
            np.testing.assert_array_equal(a, b)
    _, w_host = gpu_weights(pkg, 0, cuda_device)
    ref = orc.make_weights(0, (0, 2))
    np.testing.assert_array_equal(w_host[0][:2], ref[0][:2])
    np.testing.assert_array_equal(w_host[1][:2], ref[1][:2])
    np.testing.assert_array_equal(w_host[2][:2], ref[2][:2])
    np.testing.assert_array_equal(w_host[3][:2], ref[3][:2])


ROUTE_IN_GEMM1_CASES = [
    ("decode_t1_s3", None, None),
    ("plumbing_t16", None, None),
    ("small_t64", None, 7),         # T < 8: some waves route no token
    ("small_t64", 224, 16),         # last routing group local
    ("prefill_t1024", 256, 5),      # no local expert at all
]


@pytest.mark.parametrize("name,offset,T", ROUTE_IN_GEMM1_CASES)
def test_routing_inside_gemm1_matches_route_kernel(pkg, cuda_device, name, offset, T):
    """T <= 16: the layer routes inside GEMM1 (every workgroup from LDS,
    workgroup 0 writing the results); the workspace routing results equal the
    routing-only entry point's bit for bit."""
    cfg = pkg.synth.CONFIGS[name]
    off = cfg.local_expert_offset if offset is None else offset
    w, _ = gpu_weights(pkg, cfg.seed, cuda_device)
    tok, _ = gpu_tokens(pkg, cfg, cuda_device, T)
    T = tok[0].shape[0]
    assert T <= 16
    print(f"routing-in-GEMM1 case {name} offset={off} T={T}", flush=True)
    run_layer(pkg, tok, w, off, cfg.routed_scaling_factor)
    lay = pkg.intermediates(pkg.workspace(cuda_device, T), T)
    n = int(lay.expert_off[32].item())
    got = [x.clone() for x in (lay.topk_ids, lay.topk_w, lay.pair_row, lay.expert_off, lay.perm_token[:n], lay.perm_w[:n])]
    ws = torch.empty_like(pkg.workspace(cuda_device, T))
    r = pkg.route(tok[0], tok[1], off, cfg.routed_scaling_factor, ws=ws)
    torch.cuda.synchronize()
    exp = (r.topk_ids, r.topk_w, r.pair_row, r.expert_off, r.perm_token[:n], r.perm_w[:n])
    for name_, g, e in zip(("ids", "w", "pair_row", "expert_off", "perm_token", "perm_w"), got, exp):
        assert torch.equal(g, e), f"{name_} differs"
