"""GPU parity of the routing + permutation kernel (route.hip) against the
oracle's restatement of moe.py:123-179, through the C ABI."""
import numpy as np
import pytest
import torch

from util import gpu_tokens, near_tie_tokens

pytestmark = pytest.mark.gpu

CASES = [
    ("plumbing_t16", None, None),
    ("decode_t1", None, None),
    ("decode_t1_s3", None, None),
    ("small_t64", None, None),
    ("prefill_t1024", None, None),
    ("skewed_t8192", None, None),
    ("prefill_t1024", 224, None),   # last routing group local
    ("prefill_t1024", 240, None),   # window partly past expert 255
    ("prefill_t1024", -16, None),   # window partly below expert 0
    ("prefill_t1024", 256, None),   # no local expert at all
    ("small_t64", 96, 3),           # T not a multiple of the 4-token block
    ("small_t64", None, 17),        # one workgroup routes and permutes (T <= 24)
    ("prefill_t1024", None, 24),    # largest T of the one-workgroup routing
    ("prefill_t1024", None, 25),    # smallest T of routing plus a permutation launch
    ("skewed_t8192", 64, 777),      # ragged, large
    # permutation workgroup shapes: one wave (T <= 64), 128-token chunks
    # (64 < T <= 1024), 1024-token chunks beyond
    ("prefill_t1024", None, 64),
    ("prefill_t1024", None, 65),
    ("prefill_t1024", None, 129),
    ("skewed_t8192", None, 1025),
]


def expected_perm(ids, offset):
    """Rows of each local expert in ascending token order (moe.py:174-178)."""
    T = ids.shape[0]
    lists = [[] for _ in range(32)]
    for t in range(T):
        for e in ids[t]:
            le = int(e) - offset
            if 0 <= le < 32:
                lists[le].append(t)
    return lists


@pytest.mark.parametrize("name,offset,T", CASES)
def test_route_matches_oracle(pkg, orc, cuda_device, name, offset, T):
    cfg = pkg.synth.CONFIGS[name]
    off = cfg.local_expert_offset if offset is None else offset
    tok, host = gpu_tokens(pkg, cfg, cuda_device, T)
    print(f"route case {name} offset={off} T={tok[0].shape[0]}", flush=True)
    check_route(pkg, orc, tok, host, off, cfg.routed_scaling_factor)


# More logits and biases: the generator's seeds 10-25 (none is a config's own),
# each with another local window, so that many more score patterns meet the
# ranking, the near-tie rule and the permutation.
SEED_SWEEP = [(s, 32 * (s % 8)) for s in range(10, 26)]


@pytest.mark.parametrize("seed,offset", SEED_SWEEP)
def test_route_seed_sweep(pkg, orc, cuda_device, seed, offset):
    cfg = pkg.synth.CONFIGS["prefill_t1024"]
    tok = pkg.synth.tokens(cfg, cuda_device, 512, seed=seed)
    host = (tok[0].cpu().numpy(), tok[1].view(torch.int16).cpu().numpy().view(np.uint16))
    print(f"route seed sweep seed={seed} offset={offset} T=512", flush=True)
    check_route(pkg, orc, tok, host, offset, cfg.routed_scaling_factor)


# Other routed scaling factors on each routing implementation: T = 1 and 16
# (single-token and one-workgroup paths), 24 / 25 (either side of the
# one-launch limit) and 300 (route kernel + permutation).
RSF_ROUTE_CASES = [(T, rsf) for T in (1, 16, 24, 25, 300) for rsf in (1.0, 0.37, 7.0)]


@pytest.mark.parametrize("T,rsf", RSF_ROUTE_CASES)
def test_route_other_scaling_factors(pkg, orc, cuda_device, T, rsf):
    cfg = pkg.synth.CONFIGS["prefill_t1024"]
    tok = pkg.synth.tokens(cfg, cuda_device, T)
    host = (tok[0].cpu().numpy(), tok[1].view(torch.int16).cpu().numpy().view(np.uint16))
    print(f"route rsf case T={T} rsf={rsf}", flush=True)
    check_route(pkg, orc, tok, host, cfg.local_expert_offset, rsf)


def check_route(pkg, orc, tok, host, off, rsf):
    """Expert ids equal the oracle's (moe.py:123-158) outside near-ties of the
    fp32 scores, weights bit-exact where the ids agree, and the permutation is
    the oracle's (ascending token order per expert, moe.py:174-178)."""
    T = tok[0].shape[0]
    r = pkg.route(tok[0], tok[1], off, rsf)
    torch.cuda.synchronize()
    ids = r.topk_ids.cpu().numpy()
    w = r.topk_w.cpu().numpy()
    ref_ids, ref_w = orc.route(host[0], host[1], rsf)

    # ids ascending per token, 8 distinct
    assert (np.diff(ids, axis=1) > 0).all()
    tie = near_tie_tokens(host[0], host[1], rsf)
    same = (ids == ref_ids).all(axis=1)
    mismatch = np.nonzero(~same & ~tie)[0]
    assert mismatch.size == 0, f"expert ids differ at tokens {mismatch[:8]}"
    assert tie.sum() <= max(2, T // 500), f"unexpectedly many near-ties: {tie.sum()}"
    # weights: same op order as the oracle -> bit-exact where ids agree
    np.testing.assert_array_equal(w[same], ref_w[same])

    # permutation (deterministic: ascending token order inside each expert)
    exp = expected_perm(ids, off)
    offs = r.expert_off.cpu().numpy()
    counts = np.array([len(x) for x in exp])
    np.testing.assert_array_equal(offs, np.concatenate([[0], np.cumsum(counts)]))
    perm = r.perm_token.cpu().numpy()
    for le in range(32):
        np.testing.assert_array_equal(perm[offs[le]:offs[le + 1]], exp[le])
    pair = r.pair_row.cpu().numpy()
    pw = r.perm_w.cpu().numpy()
    for t in range(T):
        for k in range(8):
            le = int(ids[t, k]) - off
            if 0 <= le < 32:
                row = pair[t, k]
                assert offs[le] <= row < offs[le + 1] and perm[row] == t
                assert pw[row] == w[t, k]
            else:
                assert pair[t, k] == -1
    # per-workgroup histograms (the two-launch path, T > 24) add up to the
    # expert counts
    if T > pkg.moe.ROUTE_ONE_WORKGROUP_MAX_TOKENS:
        np.testing.assert_array_equal(r.block_hist.cpu().numpy().sum(axis=0), counts)
    else:
        assert r.block_hist is None


def test_route_repeatable(pkg, cuda_device):
    cfg = pkg.synth.CONFIGS["skewed_t8192"]
    tok, _ = gpu_tokens(pkg, cfg, cuda_device)
    a = pkg.route(tok[0], tok[1], 0, 2.5)
    snap = [x.clone() for x in (a.topk_ids, a.topk_w, a.pair_row, a.expert_off, a.perm_token)]
    b = pkg.route(tok[0], tok[1], 0, 2.5)
    for x, y in zip(snap, (b.topk_ids, b.topk_w, b.pair_row, b.expert_off, b.perm_token)):
        assert torch.equal(x, y)


@pytest.mark.parametrize("T", [1, 16, 40])
def test_exact_ties_go_to_lower_ids(pkg, cuda_device, T):
    """Exact score ties are exempt from the reference parity above (torch.topk
    resolves them through nth_element). The GPU resolves them
    deterministically to the lower group and expert index. With all scores
    equal, groups 0-3 are kept and experts 0-7 are chosen with equal weights.
    Covers the single-workgroup (T <= 16) and the multi-workgroup path."""
    print(f"exact-ties case T={T}", flush=True)
    logits = torch.zeros((T, 256), dtype=torch.float32, device=cuda_device)
    bias = torch.zeros(256, dtype=torch.bfloat16, device=cuda_device)
    r = pkg.route(logits, bias, 0, 2.5)
    torch.cuda.synchronize()
    ids = r.topk_ids.cpu()
    assert (ids == torch.arange(8, dtype=torch.int32)).all()
    w = r.topk_w.cpu()
    assert (w == w[0, 0]).all() and abs(float(w[0, 0]) - 2.5 / 8) < 1e-6


def test_single_token_routing_matches_per_wave_routing(pkg, cuda_device):
    """T = 1 routes in a single workgroup with four waves, its top-8 found by
    a threshold and a rank over the candidates (route_one); T > 16 routes
    each token on one wave with eight rounds of a wave maximum (route_token).
    Both restate moe.py:123-158 and must agree bit for bit on the same rows:
    rows of two synthetic configs (hot experts with a +2 bias among them),
    rows of a few distinct values (exact ties of keys and of group scores),
    rows whose top twelve logits are equal (tied candidates of the rank),
    and all-equal rows (every key ties: more than 16 candidates, which take
    the eight rounds)."""
    print("single-token routing against per-wave routing", flush=True)
    sk = pkg.synth.CONFIGS["skewed_t8192"]
    pf = pkg.synth.CONFIGS["prefill_t1024"]
    tok_sk, _ = gpu_tokens(pkg, sk, cuda_device, 384)
    tok_pf, _ = gpu_tokens(pkg, pf, cuda_device, 256)
    g = torch.Generator().manual_seed(11)
    ties = (torch.randint(0, 4, (256, 256), generator=g).float() * 0.25).to(cuda_device)
    # twelve experts per row share the top logit: about a dozen tied
    # candidates (the rank, with ties to break by expert)
    top = torch.randn((128, 256), generator=g) * 0.5
    for row in top:
        row[torch.randperm(256, generator=g)[:12]] = 3.0
    top = top.to(cuda_device)
    flat = torch.full((4, 256), 0.5, device=cuda_device)
    for bias in (tok_sk[1], tok_pf[1], torch.zeros_like(tok_pf[1])):
        logits = torch.cat([tok_sk[0], tok_pf[0], ties, top, flat]).contiguous()
        n = logits.shape[0]
        ws = torch.empty_like(pkg.workspace(cuda_device, n))
        whole = pkg.route(logits, bias, 0, 2.5, ws=ws)
        ids_all, w_all = whole.topk_ids.clone(), whole.topk_w.clone()
        ids_one = torch.empty_like(ids_all)
        w_one = torch.empty_like(w_all)
        ws1 = torch.empty_like(pkg.workspace(cuda_device, 1))
        for t in range(n):
            r = pkg.route(logits[t:t + 1], bias, 0, 2.5, ws=ws1)
            ids_one[t] = r.topk_ids[0]
            w_one[t] = r.topk_w[0]
        torch.cuda.synchronize()
        bad = (ids_one != ids_all).any(dim=1) | (w_one.view(torch.int32) != w_all.view(torch.int32)).any(dim=1)
        assert not bad.any(), f"{int(bad.sum())} of {n} rows differ, first {int(bad.nonzero()[0])}"
