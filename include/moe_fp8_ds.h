/*
 * moe_fp8_ds.h -- C ABI of the MI355X (gfx950) FP8 block-scale MoE layer
 * `moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048`.
 *
 * Drop-in for the contest solution's operator entry point
 *   moe/solution/cuda/moe.cu:2650-2661  run_impl(routing_logits, routing_bias,
 *     hidden_states, hidden_states_scale, gemm1_weights, gemm1_weights_scale,
 *     gemm2_weights, gemm2_weights_scale, local_expert_offset,
 *     routed_scaling_factor, output)
 * exported as `run` (moe.cu:2898, entry "moe.cu::run" in moe/config.toml:8,
 * destination-passing style).  The ABI keeps the argument order and meaning
 * and replaces the tvm-ffi TensorViews with plain device pointers plus T, and
 * adds an explicit caller-owned workspace and HIP stream.
 *
 * Layouts (all row-major, contiguous, device memory):
 *   routing_logits       float32   [T, 256]
 *   routing_bias         bfloat16  [256]
 *   hidden_states        e4m3fn    [T, 7168]
 *   hidden_states_scale  float32   [56, T]          (transposed: [H/128, T])
 *   gemm1_weights        e4m3fn    [32, 4096, 7168]
 *   gemm1_weights_scale  float32   [32, 32, 56]
 *   gemm2_weights        e4m3fn    [32, 7168, 2048]
 *   gemm2_weights_scale  float32   [32, 56, 16]
 *   output               bfloat16  [T, 7168]        (every element written)
 *
 * All entry points are stream-ordered on `stream`, never synchronise the host
 * and never allocate.  Two calls may run concurrently only with distinct
 * workspaces.  Every entry point returns a moe_fp8_ds_status (0 = success)
 * and validates its arguments before launching anything.
 */
#ifndef MOE_FP8_DS_H
#define MOE_FP8_DS_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_FP8_DS_VERSION 1

typedef enum {
  MOE_FP8_DS_OK = 0,
  MOE_FP8_DS_ERR_NULL = -1,      /* a required pointer is NULL                 */
  MOE_FP8_DS_ERR_SHAPE = -2,     /* T < 0 or T > moe_fp8_ds_max_tokens()       */
  MOE_FP8_DS_ERR_ALIGN = -3,     /* a pointer is not 16-byte aligned           */
  MOE_FP8_DS_ERR_WORKSPACE = -4, /* workspace smaller than workspace_size(T)   */
  MOE_FP8_DS_ERR_HIP = -5,       /* a HIP launch failed                        */
  MOE_FP8_DS_ERR_ARG = -6,       /* non-finite routed_scaling_factor           */
  MOE_FP8_DS_ERR_SCRATCH = -7    /* T > MOE_FP8_DS_NOALLOC_MAX_TOKENS (moe_fp8_ds_run_noalloc) */
} moe_fp8_ds_status;

/* Library version (MOE_FP8_DS_VERSION of the build). */
int moe_fp8_ds_version(void);

/* Human-readable text of a status code (static storage). */
const char* moe_fp8_ds_status_string(int status);

/* Largest T accepted by the entry points. */
int64_t moe_fp8_ds_max_tokens(void);

/* Bytes of workspace `moe_fp8_ds_run` needs for T tokens.  The workspace needs
 * no initialisation and carries no state between calls.  Replaces the
 * reference's lazily grown process-global workspace
 * (moe/solution/cuda/moe.cu:2511-2589). */
size_t moe_fp8_ds_workspace_size(int64_t T);

/* The whole layer (moe.cu:2650-2896 / moe.py:28-202): routing, permutation,
 * FP8 GEMM1 + SwiGLU, GEMM2, weighted combine, bf16 output.  T == 0 is a
 * successful no-op.  Expert ids outside [0, 256) of the local window
 * [local_expert_offset, local_expert_offset + 32) contribute nothing, as in
 * moe.py:169-171. */
int moe_fp8_ds_run(const float* routing_logits, const void* routing_bias,
                   const void* hidden_states, const float* hidden_states_scale,
                   const void* gemm1_weights, const float* gemm1_weights_scale,
                   const void* gemm2_weights, const float* gemm2_weights_scale,
                   int64_t local_expert_offset, double routed_scaling_factor, void* output,
                   int64_t T, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Largest T moe_fp8_ds_run_noalloc accepts. */
#define MOE_FP8_DS_NOALLOC_MAX_TOKENS 64

/* moe_fp8_ds_run without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference, whose
 * run_impl grows a hidden global workspace with cudaMalloc
 * (moe/solution/cuda/moe.cu:2511-2589).
 *
 * The intermediates live in a static device array inside the library, sized
 * for MOE_FP8_DS_NOALLOC_MAX_TOKENS tokens (decode and small batches; the
 * workspace size for 64 tokens, about 4.2 MB, held on every device the library runs on until the process ends).
 * T above that returns MOE_FP8_DS_ERR_SCRATCH.  The call allocates nothing
 * and, like moe_fp8_ds_run, needs no initialised scratch.  It uses the
 * scratch of the current device (the stream must belong to it), and every
 * call on one device shares that scratch: calls that overlap on one device
 * (concurrent streams or host threads) race and must be serialised by the
 * caller.  Results are bit-identical to moe_fp8_ds_run's. */
int moe_fp8_ds_run_noalloc(const float* routing_logits, const void* routing_bias,
                           const void* hidden_states, const float* hidden_states_scale,
                           const void* gemm1_weights, const float* gemm1_weights_scale,
                           const void* gemm2_weights, const float* gemm2_weights_scale,
                           int64_t local_expert_offset, double routed_scaling_factor, void* output,
                           int64_t T, hipStream_t stream);

/* Number of device stages of moe_fp8_ds_run: routing + permutation, GEMM1 +
 * SwiGLU, GEMM2, combine.  For T <= 16 the routing runs inside GEMM1 (stage 0
 * is empty), and for T <= 64 the combine inside GEMM2 (stage 3 is empty). */
#define MOE_FP8_DS_NUM_STAGES 4

/* moe_fp8_ds_run, plus a hipEventRecord on `stream` before the first stage and
 * after each stage: stage_events[0..MOE_FP8_DS_NUM_STAGES], all created by the
 * caller (timing-enabled).  Elapsed time between events i and i+1 is stage i.
 * Instrumentation for benchmarks; it has no counterpart in the reference
 * (whose harness times only the whole call, moe/scripts/run_local.py:33). */
int moe_fp8_ds_run_profiled(const float* routing_logits, const void* routing_bias,
                            const void* hidden_states, const float* hidden_states_scale,
                            const void* gemm1_weights, const float* gemm1_weights_scale,
                            const void* gemm2_weights, const float* gemm2_weights_scale,
                            int64_t local_expert_offset, double routed_scaling_factor, void* output,
                            int64_t T, void* workspace, size_t workspace_bytes, hipStream_t stream,
                            hipEvent_t* stage_events);

/* Routing and permutation only (moe.py:123-158 and the per-expert token lists
 * of moe.py:168-179; moe.cu route_kernel :60-186, scan :217-283, perm_fill
 * :288-309).  Fills the workspace regions described by
 * moe_fp8_ds_workspace_layout; used by kernel-level parity tests. */
int moe_fp8_ds_route(const float* routing_logits, const void* routing_bias,
                     int64_t local_expert_offset, double routed_scaling_factor, int64_t T,
                     void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Byte offsets of the intermediates inside the workspace for T tokens. */
typedef struct {
  size_t topk_ids;   /* int32 [T, 8]   selected global expert ids, ascending     */
  size_t topk_w;     /* float [T, 8]   combination weights (same order)          */
  size_t pair_row;   /* int32 [T, 8]   permuted row of each pair, -1 if not local */
  size_t expert_off; /* int32 [33]     row offsets per local expert; [32] = N_sel */
  size_t perm_token; /* int32 [8T]     token of each permuted row                 */
  size_t perm_w;     /* float [8T]     combination weight of each permuted row    */
  size_t act;        /* bf16 pairs [8T, 4096]: SwiGLU output rows, value = hi + lo;
                        per 64-column chunk c, 64 hi then 64 lo bf16 (8 KB/row).
                        T >= 1024 with two or more local experts that every token
                        selects: their rows times the routing weight              */
  size_t down;       /* float [8T, 7168] GEMM2 output rows (T > 64 only; for
                        T <= 64 GEMM2 combines in registers and the region is empty).
                        Experts every token selects (as for act): the first one's
                        rows hold each token's weighted sum over all of them, the
                        others' rows are not written                              */
  size_t block_hist; /* int32 [workgroups, 32] local-expert pairs per routing workgroup
                        (T > 16; ceil(T/4) workgroups up to T = 1024, ceil(T/16) beyond) */
  size_t total;      /* = moe_fp8_ds_workspace_size(T)                            */
} moe_fp8_ds_layout;

int moe_fp8_ds_workspace_layout(int64_t T, moe_fp8_ds_layout* layout);

/* The step before the layer.  No counterpart in the reference, which only
 * consumes its result: hidden_states [T,7168] e4m3 and hidden_states_scale
 * [56,T] fp32 (moe.py:32-33, moe.cu:2650-2661).  Quantises bf16 hidden rows
 * [T,7168] per 128-column block: scale = absmax/448 (1 for an all-zero
 * block; NaN does not enter the absmax), q = e4m3(x/scale) rounded to nearest
 * even and saturated to +-448; scales are written transposed, [56,T].
 * hidden_bf16 and hidden_fp8 must be 16-byte aligned, hidden_scale 4-byte.  Stream
 * ordered, no allocation, T == 0 is a no-op. */
int moe_fp8_ds_quantize_hidden(const void* hidden_bf16, int64_t T, void* hidden_fp8, float* hidden_scale,
                               hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
