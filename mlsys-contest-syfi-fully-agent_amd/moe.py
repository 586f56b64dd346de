"""Python entry point of the gfx950 FP8 MoE layer, mirroring the contest
solution's operator `run` (moe/solution/cuda/moe.cu:2650-2661, exported at
moe.cu:2898 as "moe.cu::run", destination-passing style per moe/config.toml:6-11).

    run(routing_logits, routing_bias, hidden_states, hidden_states_scale,
        gemm1_weights, gemm1_weights_scale, gemm2_weights, gemm2_weights_scale,
        local_expert_offset, routed_scaling_factor, output)

Arguments have the names, order, dtypes and shapes of the definition
(full-agent-pipeline/references/moe.py:29-40, shape checks moe.py:71-91); the
result is written into `output` ([T, 7168] bf16), which is also returned.
Shape and dtype mismatches raise AssertionError like the reference's asserts;
a failing HIP call raises RuntimeError.  The work is enqueued on the current
HIP stream of the tensors' device; nothing synchronises the host.

All arithmetic happens in libmoe_fp8_ds.so (HIP kernels for gfx950); this file
only checks arguments, owns a workspace per (device, stream) and passes pointers.
"""
from __future__ import annotations

import threading
from collections import OrderedDict

import torch

from . import _lib

H, I, E_LOCAL, E_GLOBAL, TOP_K, BLOCK = 7168, 2048, 32, 256, 8, 128
# Up to this T the GEMM2 kernel also performs the weighted combine and the
# workspace holds no GEMM2 rows (`down`; kGemm2StreamMaxTokens in
# csrc/moe_common.hpp).
FUSED_COMBINE_MAX_TOKENS = 64
# Up to this T one workgroup routes the tokens and builds the permutation
# (inside GEMM1 for T <= 16 in the layer), so the workspace holds no
# per-workgroup routing histograms (`block_hist`; kRouteSingleMaxTokens in
# csrc/route.hip).
ROUTE_ONE_WORKGROUP_MAX_TOKENS = 24
# From this T on, local experts that every token selects (T rows each; at
# least two of them) are summed inside GEMM2: their `act` rows carry the
# routing weight, and the first one's `down` rows hold each token's weighted
# sum over all of them (the others' `down` rows are not written)
# (kEveryTokenFuseMinTokens in csrc/moe_common.hpp).
EVERY_TOKEN_FUSE_MIN_TOKENS = 1024

_ws_lock = threading.Lock()
# Workspaces by (device type, device index, stream), least recently used
# first.  At most WORKSPACE_CACHE_ENTRIES are kept: code that makes a stream
# per request no longer piles up one workspace per stream (about 2.4 GB each
# at T = 8192).
WORKSPACE_CACHE_ENTRIES = 8
_ws: "OrderedDict[tuple, torch.Tensor]" = OrderedDict()
# Buffers handed out while the stream was being captured into a graph: the
# graph writes into them on every replay, so they stay alive when the cache
# drops or outgrows them, until release_workspaces().
_ws_captured: list = []

_F8, _F32, _BF16 = torch.float8_e4m3fn, torch.float32, torch.bfloat16
# torch's raw-pointer accessor of the current stream (what
# torch.cuda.current_stream(dev).cuda_stream returns, without building a
# Stream object: ~0.2 against ~1.9 us a call)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    """Raw HIP stream handle of the current torch stream of `device`."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def workspace(device: torch.device, T: int, stream: int | None = None) -> torch.Tensor:
    """Workspace of the current stream of `device`, grown on demand (needs no
    initialisation).  One buffer per (device, stream): calls on different
    streams never share one (the C entry points need distinct workspaces for
    concurrent calls), and a buffer is allocated on the stream that uses it,
    so when it grows, torch's caching allocator hands the old memory out
    again only to later work on that same stream.  The cache keeps the
    WORKSPACE_CACHE_ENTRIES most recently used streams' buffers; a buffer
    handed out during graph capture is also kept for the graph's replays
    (see release_workspaces)."""
    need = _lib.moe_lib().moe_fp8_ds_workspace_size(T)
    key = (device.type, device.index, _stream(device) if stream is None else stream)
    capturing = device.type == "cuda" and torch.cuda.is_current_stream_capturing()
    with _ws_lock:
        buf = _ws.get(key)
        if buf is None or buf.numel() < need:
            buf = torch.empty(max(need, 1 << 20), dtype=torch.uint8, device=device)
            _ws[key] = buf
        _ws.move_to_end(key)
        if capturing and not any(b is buf for b in _ws_captured):
            _ws_captured.append(buf)
        while len(_ws) > WORKSPACE_CACHE_ENTRIES:
            _ws.popitem(last=False)
        return buf


def release_workspaces() -> None:
    """Drops every cached workspace, including those kept for captured graphs:
    call it only once no graph that ran the layer will be replayed again."""
    with _ws_lock:
        _ws.clear()
        _ws_captured.clear()


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()  # the ctypes signatures (c_void_p) take plain ints


def _check(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
           gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, output=None) -> int:
    T = routing_logits.shape[0]
    assert routing_logits.dtype == _F32 and routing_logits.shape == (T, E_GLOBAL)
    assert routing_bias.dtype == _BF16 and routing_bias.shape[-1] == E_GLOBAL
    assert routing_bias.numel() == E_GLOBAL
    if hidden_states is not None:
        assert hidden_states.dtype == _F8 and hidden_states.shape == (T, H)
        assert hidden_states_scale.dtype == _F32 and hidden_states_scale.shape == (H // BLOCK, T)
        assert gemm1_weights.dtype == _F8 and gemm1_weights.shape == (E_LOCAL, 2 * I, H)
        assert gemm1_weights_scale.dtype == _F32
        assert gemm1_weights_scale.shape == (E_LOCAL, 2 * I // BLOCK, H // BLOCK)
        assert gemm2_weights.dtype == _F8 and gemm2_weights.shape == (E_LOCAL, H, I)
        assert gemm2_weights_scale.dtype == _F32
        assert gemm2_weights_scale.shape == (E_LOCAL, H // BLOCK, I // BLOCK)
    if output is not None:
        assert output.dtype == _BF16 and output.shape == (T, H)
    # one device (index -1: the CPU) and contiguous storage for every tensor
    idx = routing_logits.get_device()
    for t in (routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
              gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, output):
        if t is None:
            continue
        assert t.get_device() == idx, "all tensors must be on the same device"
        assert t.is_contiguous(), "all tensors must be contiguous"
    if not routing_logits.is_cuda:
        raise RuntimeError("moe_fp8_ds runs on a ROCm GPU only (no CPU path)")
    return T


def run(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
        gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset,
        routed_scaling_factor, output, stage_events=None):
    """`stage_events` (optional, an _lib.EventPool slice pointer) makes the
    call record MOE_FP8_DS_NUM_STAGES + 1 events around its device stages."""
    T = _check(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
               gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, output)
    dev = routing_logits.device
    stream = _stream(dev)
    ws = workspace(dev, T, stream)
    args = (routing_logits.data_ptr(), routing_bias.data_ptr(), hidden_states.data_ptr(),
            hidden_states_scale.data_ptr(), gemm1_weights.data_ptr(), gemm1_weights_scale.data_ptr(),
            gemm2_weights.data_ptr(), gemm2_weights_scale.data_ptr(), int(local_expert_offset),
            float(routed_scaling_factor), output.data_ptr(), T, ws.data_ptr(), ws.numel(), stream)
    L = _lib.moe_lib()
    if stage_events is None:
        rc = L.moe_fp8_ds_run(*args)
    else:
        rc = L.moe_fp8_ds_run_profiled(*args, stage_events)
    if rc != _lib.OK:
        raise RuntimeError(f"moe_fp8_ds_run: {_lib.status_string(rc)} ({rc})")
    return output


def run_noalloc(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
                gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset,
                routed_scaling_factor, output):
    """`run` through moe_fp8_ds_run_noalloc: no workspace, nothing allocated
    (usable under stream capture).  T <= NOALLOC_MAX_TOKENS (64); the
    library's one static scratch per device is shared by every such call, so
    overlapping calls on one device race."""
    T = _check(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
               gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, output)
    stream = _stream(routing_logits.device)
    rc = _lib.moe_lib().moe_fp8_ds_run_noalloc(
        _ptr(routing_logits), _ptr(routing_bias), _ptr(hidden_states), _ptr(hidden_states_scale),
        _ptr(gemm1_weights), _ptr(gemm1_weights_scale), _ptr(gemm2_weights), _ptr(gemm2_weights_scale),
        int(local_expert_offset), float(routed_scaling_factor), _ptr(output), T, stream)
    if rc != _lib.OK:
        raise RuntimeError(f"moe_fp8_ds_run_noalloc: {_lib.status_string(rc)} ({rc})")
    return output


def quantize_hidden(hidden_states, hidden_states_fp8=None, hidden_states_scale=None):
    """The step before the layer: bf16 hidden rows [T, 7168] -> the layer's
    `hidden_states` (e4m3, [T, 7168]) and `hidden_states_scale` (fp32, [56, T],
    transposed), one scale per 128 columns: absmax/448 (1 for an all-zero
    block), values rounded to nearest even and saturated to +-448
    (moe_fp8_ds_quantize_hidden).  Outputs are allocated unless given; the
    work is enqueued on the current stream."""
    assert hidden_states.dtype == torch.bfloat16 and hidden_states.dim() == 2 and hidden_states.shape[1] == H
    assert hidden_states.is_contiguous()
    dev = hidden_states.device
    if dev.type != "cuda":
        raise RuntimeError("moe_fp8_ds runs on a ROCm GPU only (no CPU path)")
    T = hidden_states.shape[0]
    if hidden_states_fp8 is None:
        hidden_states_fp8 = torch.empty((T, H), dtype=torch.float8_e4m3fn, device=dev)
    if hidden_states_scale is None:
        hidden_states_scale = torch.empty((H // BLOCK, T), dtype=torch.float32, device=dev)
    assert hidden_states_fp8.dtype == torch.float8_e4m3fn and hidden_states_fp8.shape == (T, H)
    assert hidden_states_scale.dtype == torch.float32 and hidden_states_scale.shape == (H // BLOCK, T)
    assert hidden_states_fp8.is_contiguous() and hidden_states_scale.is_contiguous()
    stream = _stream(dev)
    rc = _lib.moe_lib().moe_fp8_ds_quantize_hidden(_ptr(hidden_states), T, _ptr(hidden_states_fp8),
                                                   _ptr(hidden_states_scale), stream)
    if rc != _lib.OK:
        raise RuntimeError(f"moe_fp8_ds_quantize_hidden: {_lib.status_string(rc)} ({rc})")
    return hidden_states_fp8, hidden_states_scale


class RouteResult:
    """Typed views of the routing/permutation regions of a workspace."""

    def __init__(self, ws: torch.Tensor, T: int):
        lay = _lib.layout(T)

        def view(off, n, dtype):
            nbytes = n * torch.empty((), dtype=dtype).element_size()
            return ws[off:off + nbytes].view(dtype)

        self.topk_ids = view(lay.topk_ids, T * TOP_K, torch.int32).view(T, TOP_K)
        self.topk_w = view(lay.topk_w, T * TOP_K, torch.float32).view(T, TOP_K)
        self.pair_row = view(lay.pair_row, T * TOP_K, torch.int32).view(T, TOP_K)
        self.expert_off = view(lay.expert_off, E_LOCAL + 1, torch.int32)
        self.perm_token = view(lay.perm_token, T * TOP_K, torch.int32)
        self.perm_w = view(lay.perm_w, T * TOP_K, torch.float32)
        # SwiGLU rows as bf16 (hi, lo) pairs: per 64-column chunk, 64 hi then
        # 64 lo values (act_values() decodes them to fp32 hi + lo); see
        # EVERY_TOKEN_FUSE_MIN_TOKENS for the rows of experts every token selects
        self.act = view(lay.act, T * TOP_K * 2 * I, torch.int16).view(T * TOP_K, 2 * I)
        # fp32 GEMM2 rows, in the workspace only where a combine pass reads them
        self.down = (view(lay.down, T * TOP_K * H, torch.float32).view(T * TOP_K, H)
                     if T > FUSED_COMBINE_MAX_TOKENS else None)
        # one row per routing workgroup: 4 tokens each up to T = 1024, 16 beyond
        # (written only where a permutation launch reads them)
        blocks = (T + 3) // 4 if T <= 1024 else (T + 15) // 16
        self.block_hist = (view(lay.block_hist, blocks * E_LOCAL, torch.int32).view(-1, E_LOCAL)
                           if T > ROUTE_ONE_WORKGROUP_MAX_TOKENS else None)


def route(routing_logits, routing_bias, local_expert_offset, routed_scaling_factor, ws=None):
    """Routing + permutation only; returns typed views into the workspace."""
    T = _check(routing_logits, routing_bias, None, None, None, None, None, None)
    dev = routing_logits.device
    stream = _stream(dev)
    ws = workspace(dev, T, stream) if ws is None else ws
    rc = _lib.moe_lib().moe_fp8_ds_route(_ptr(routing_logits), _ptr(routing_bias), int(local_expert_offset),
                                         float(routed_scaling_factor), T, _ptr(ws), ws.numel(), stream)
    if rc != _lib.OK:
        raise RuntimeError(f"moe_fp8_ds_route: {_lib.status_string(rc)} ({rc})")
    return RouteResult(ws, T)


def act_values(act_rows: torch.Tensor) -> torch.Tensor:
    """fp32 values [n, 2048] of act rows [n, 4096] (int16 bf16 bits, per
    64-column chunk 64 hi then 64 lo): hi + lo."""
    n = act_rows.shape[0]
    bits = act_rows.reshape(n, I // 64, 2, 64).to(torch.int32) & 0xFFFF
    f = (bits << 16).view(torch.float32)
    return (f[:, :, 0, :] + f[:, :, 1, :]).reshape(n, I)


def intermediates(ws: torch.Tensor, T: int) -> RouteResult:
    """Views of every intermediate region after a `run` call for T tokens."""
    return RouteResult(ws, T)
