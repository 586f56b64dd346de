"""The Python mirror's workspace cache: bounded however many streams call the
layer, and a buffer that a captured graph writes into stays alive after the
cache outgrows or drops it."""
import pytest
import torch

from util import gpu_tokens, gpu_weights

pytestmark = pytest.mark.gpu

H = 7168


def _out(T, dev):
    return torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=dev)


def test_cache_bounded_over_many_streams(pkg, cuda_device):
    """A new stream per call (a serving loop that makes streams per request)
    keeps at most WORKSPACE_CACHE_ENTRIES buffers; every call gives the same
    bits."""
    cfg = pkg.synth.CONFIGS["prefill_t1024"]
    w, _ = gpu_weights(pkg, cfg.seed, cuda_device)
    T = 96
    tok, _ = gpu_tokens(pkg, cfg, cuda_device, T)
    pkg.release_workspaces()
    ref = _out(T, cuda_device)
    pkg.run(*tok, *w, cfg.local_expert_offset, cfg.routed_scaling_factor, ref)
    torch.cuda.synchronize()
    ws_bytes = pkg.workspace(cuda_device, T).numel()
    base = torch.cuda.memory_allocated(cuda_device)
    cap = pkg.moe.WORKSPACE_CACHE_ENTRIES
    for i in range(3 * cap):
        s = torch.cuda.Stream(device=cuda_device)
        out = _out(T, cuda_device)
        with torch.cuda.stream(s):
            pkg.run(*tok, *w, cfg.local_expert_offset, cfg.routed_scaling_factor, out)
        s.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"stream {i}"
        assert len(pkg.moe._ws) <= cap
        del out
    torch.cuda.synchronize()
    grown = torch.cuda.memory_allocated(cuda_device) - base
    print(f"workspace {ws_bytes} B, cache {len(pkg.moe._ws)} entries, allocated +{grown} B after {3 * cap} streams")
    assert grown <= cap * ws_bytes
    pkg.release_workspaces()
    assert len(pkg.moe._ws) == 0


def test_captured_workspace_outlives_growth(pkg, cuda_device):
    """A graph captures the layer at T = 80; a larger eager call on the same
    stream then grows that stream's workspace.  Every replay still gives the
    eager T = 80 bits: the captured buffer was kept, not handed out again."""
    cfg = pkg.synth.CONFIGS["prefill_t1024"]
    w, _ = gpu_weights(pkg, cfg.seed, cuda_device)
    small, _ = gpu_tokens(pkg, cfg, cuda_device, 80)
    big, _ = gpu_tokens(pkg, cfg, cuda_device, 700)
    pkg.release_workspaces()
    ref = _out(80, cuda_device)
    pkg.run(*small, *w, cfg.local_expert_offset, cfg.routed_scaling_factor, ref)
    torch.cuda.synchronize()

    s = torch.cuda.Stream(device=cuda_device)
    got = _out(80, cuda_device)
    with torch.cuda.stream(s):
        pkg.run(*small, *w, cfg.local_expert_offset, cfg.routed_scaling_factor, got)  # eager warm-up on s
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        pkg.run(*small, *w, cfg.local_expert_offset, cfg.routed_scaling_factor, got)
    torch.cuda.synchronize()
    assert len(pkg.moe._ws_captured) >= 1
    big_out = _out(700, cuda_device)
    for rep in range(3):
        got.fill_(float("nan"))
        # eager work between the replays: a larger call that grows the
        # capture stream's workspace, and an allocation that could reuse
        # freed memory
        with torch.cuda.stream(s):
            pkg.run(*big, *w, cfg.local_expert_offset, cfg.routed_scaling_factor, big_out)
            junk = torch.full((1 << 22,), 7, dtype=torch.int32, device=cuda_device)
        s.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"captured-workspace replay {rep}", flush=True)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"replay {rep}"
        del junk
    del graph
    pkg.release_workspaces()


@pytest.mark.parametrize("name,T", [("small_t64", 1100), ("skewed_t8192", 1025)])
def test_graph_replay_with_both_gemm1_kernels(pkg, cuda_device, name, T):
    """For 1,025-1,536 tokens the layer launches both GEMM1 kernels and the
    row counts choose one (the tiled kernel for spread rows, the wide one for
    hot experts).  A graph of such a call replays to the eager bits, with
    eager work between the replays."""
    cfg = pkg.synth.CONFIGS[name]
    w, _ = gpu_weights(pkg, cfg.seed, cuda_device)
    tok, _ = gpu_tokens(pkg, cfg, cuda_device, T)
    print(f"graph case {name} T={T}", flush=True)
    ref = _out(T, cuda_device)
    pkg.run(*tok, *w, cfg.local_expert_offset, cfg.routed_scaling_factor, ref)
    torch.cuda.synchronize()
    s = torch.cuda.Stream(device=cuda_device)
    got = _out(T, cuda_device)
    with torch.cuda.stream(s):
        pkg.run(*tok, *w, cfg.local_expert_offset, cfg.routed_scaling_factor, got)  # eager warm-up on s
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        pkg.run(*tok, *w, cfg.local_expert_offset, cfg.routed_scaling_factor, got)
    torch.cuda.synchronize()
    for rep in range(3):
        got.fill_(float("nan"))
        junk = torch.full((1 << 20,), 3, dtype=torch.int32, device=cuda_device)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"replay {rep}"
        del junk
    del graph
    pkg.release_workspaces()
