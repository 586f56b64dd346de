// moe_api.cpp -- the C ABI (include/moe_fp8_ds.h): argument validation,
// workspace layout and the stream-ordered launch sequence.
//
// Replaces the reference host path run_impl (moe/solution/cuda/moe.cu:2650-2896):
// no lazily grown global workspace (the caller owns it), no default-stream use
// (the caller's stream), no host synchronisation at any T (the device builds
// the expert schedule), and status codes instead of unchecked CUDA calls.
#include <cmath>
#include <mutex>

#include "../../include/moe_fp8_ds.h"
#include "kernels.hpp"

namespace {

// ---- scratch of the no-allocation entry point -----------------------------
// moe_fp8_ds_run_noalloc keeps its intermediates in this file-scope device
// array instead of a caller workspace: the layer's workspace layout for
// MOE_FP8_DS_NOALLOC_MAX_TOKENS tokens.  Each device the library runs on
// holds its own copy (loaded with the code object) until the process ends.
// In host code `scratch` only names the symbol; its device address comes from
// hipGetSymbolAddress, once per device (noalloc_scratch).
constexpr size_t kNoAllocScratchBytes = moe::make_layout(MOE_FP8_DS_NOALLOC_MAX_TOKENS).total;
static_assert(kNoAllocScratchBytes <= (size_t)8 << 20, "the no-allocation scratch stays small");
__device__ __align__(256) char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch, looked up on the first call
// on that device; nullptr on failure.
void* noalloc_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_common(int64_t T, void* workspace, size_t workspace_bytes, double rsf) {
  if (T < 0 || T > moe::kMaxTokens) return MOE_FP8_DS_ERR_SHAPE;
  if (!std::isfinite(rsf)) return MOE_FP8_DS_ERR_ARG;
  if (T == 0) return MOE_FP8_DS_OK;
  if (!workspace) return MOE_FP8_DS_ERR_NULL;
  if (!aligned16(workspace)) return MOE_FP8_DS_ERR_ALIGN;
  if (workspace_bytes < moe::make_layout(T).total) return MOE_FP8_DS_ERR_WORKSPACE;
  return MOE_FP8_DS_OK;
}

}  // namespace

extern "C" {

int moe_fp8_ds_version(void) { return MOE_FP8_DS_VERSION; }

const char* moe_fp8_ds_status_string(int status) {
  switch (status) {
    case MOE_FP8_DS_OK: return "ok";
    case MOE_FP8_DS_ERR_NULL: return "null pointer argument";
    case MOE_FP8_DS_ERR_SHAPE: return "token count out of range";
    case MOE_FP8_DS_ERR_ALIGN: return "pointer not 16-byte aligned";
    case MOE_FP8_DS_ERR_WORKSPACE: return "workspace too small";
    case MOE_FP8_DS_ERR_HIP: return "HIP launch failed";
    case MOE_FP8_DS_ERR_ARG: return "invalid scalar argument";
    case MOE_FP8_DS_ERR_SCRATCH: return "T exceeds MOE_FP8_DS_NOALLOC_MAX_TOKENS (no-allocation entry point)";
    default: return "unknown status";
  }
}

int64_t moe_fp8_ds_max_tokens(void) { return moe::kMaxTokens; }

size_t moe_fp8_ds_workspace_size(int64_t T) {
  if (T < 0 || T > moe::kMaxTokens) return 0;
  return moe::make_layout(T).total;
}

int moe_fp8_ds_workspace_layout(int64_t T, moe_fp8_ds_layout* out) {
  if (!out) return MOE_FP8_DS_ERR_NULL;
  if (T < 0 || T > moe::kMaxTokens) return MOE_FP8_DS_ERR_SHAPE;
  const moe::Layout L = moe::make_layout(T);
  out->topk_ids = L.topk_ids;
  out->topk_w = L.topk_w;
  out->pair_row = L.pair_row;
  out->expert_off = L.expert_off;
  out->perm_token = L.perm_token;
  out->perm_w = L.perm_w;
  out->act = L.act;
  out->down = L.down;
  out->block_hist = L.block_hist;
  out->total = L.total;
  return MOE_FP8_DS_OK;
}

int moe_fp8_ds_route(const float* routing_logits, const void* routing_bias,
                     int64_t local_expert_offset, double routed_scaling_factor, int64_t T,
                     void* workspace, size_t workspace_bytes, hipStream_t stream) {
  int rc = check_common(T, workspace, workspace_bytes, routed_scaling_factor);
  if (rc != MOE_FP8_DS_OK || T == 0) return rc;
  if (!routing_logits || !routing_bias) return MOE_FP8_DS_ERR_NULL;
  if (!aligned16(routing_logits)) return MOE_FP8_DS_ERR_ALIGN;
  const moe::Layout L = moe::make_layout(T);
  hipError_t err = moe::launch_route(routing_logits, (const uint16_t*)routing_bias,
                                     (float)routed_scaling_factor, (int)T, local_expert_offset, L,
                                     (char*)workspace, stream);
  return err == hipSuccess ? MOE_FP8_DS_OK : MOE_FP8_DS_ERR_HIP;
}

static int run_layer(const float* routing_logits, const void* routing_bias, const void* hidden_states,
                     const float* hidden_states_scale, const void* gemm1_weights,
                     const float* gemm1_weights_scale, const void* gemm2_weights,
                     const float* gemm2_weights_scale, int64_t local_expert_offset,
                     double routed_scaling_factor, void* output, int64_t T, void* workspace,
                     size_t workspace_bytes, hipStream_t stream, hipEvent_t* events) {
  int rc = check_common(T, workspace, workspace_bytes, routed_scaling_factor);
  if (rc != MOE_FP8_DS_OK || T == 0) return rc;
  const void* ptrs[] = {routing_logits, routing_bias,        hidden_states,  hidden_states_scale,
                        gemm1_weights,  gemm1_weights_scale, gemm2_weights,  gemm2_weights_scale,
                        output};
  for (const void* p : ptrs)
    if (!p) return MOE_FP8_DS_ERR_NULL;
  for (const void* p : ptrs)
    if (!aligned16(p)) return MOE_FP8_DS_ERR_ALIGN;

  const moe::Layout L = moe::make_layout(T);
  char* ws = (char*)workspace;
  const int t = (int)T;
  hipError_t err = hipSuccess;
  auto mark = [&](int i) {
    if (events && err == hipSuccess) err = hipEventRecord(events[i], stream);
  };
  mark(0);
  if (err == hipSuccess && !moe::gemm1_routes(t))
    err = moe::launch_route(routing_logits, (const uint16_t*)routing_bias, (float)routed_scaling_factor, t,
                            local_expert_offset, L, ws, stream);
  mark(1);
  if (err == hipSuccess)
    err = moe::launch_gemm1((const uint8_t*)hidden_states, hidden_states_scale, t, (const uint8_t*)gemm1_weights,
                            gemm1_weights_scale, routing_logits, (const uint16_t*)routing_bias,
                            (float)routed_scaling_factor, local_expert_offset, L, ws, stream);
  mark(2);
  if (err == hipSuccess)
    err = moe::launch_gemm2(t, (const uint8_t*)gemm2_weights, gemm2_weights_scale, L, ws, output, stream);
  mark(3);
  if (err == hipSuccess && !moe::gemm2_fuses_combine(t)) err = moe::launch_combine(t, L, ws, output, stream);
  mark(4);
  return err == hipSuccess ? MOE_FP8_DS_OK : MOE_FP8_DS_ERR_HIP;
}

int moe_fp8_ds_run(const float* routing_logits, const void* routing_bias, const void* hidden_states,
                   const float* hidden_states_scale, const void* gemm1_weights,
                   const float* gemm1_weights_scale, const void* gemm2_weights,
                   const float* gemm2_weights_scale, int64_t local_expert_offset,
                   double routed_scaling_factor, void* output, int64_t T, void* workspace,
                   size_t workspace_bytes, hipStream_t stream) {
  return run_layer(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
                   gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset,
                   routed_scaling_factor, output, T, workspace, workspace_bytes, stream, nullptr);
}

int moe_fp8_ds_run_profiled(const float* routing_logits, const void* routing_bias,
                            const void* hidden_states, const float* hidden_states_scale,
                            const void* gemm1_weights, const float* gemm1_weights_scale,
                            const void* gemm2_weights, const float* gemm2_weights_scale,
                            int64_t local_expert_offset, double routed_scaling_factor, void* output,
                            int64_t T, void* workspace, size_t workspace_bytes, hipStream_t stream,
                            hipEvent_t* stage_events) {
  if (!stage_events) return MOE_FP8_DS_ERR_NULL;
  for (int i = 0; i < MOE_FP8_DS_NUM_STAGES + 1; ++i)
    if (!stage_events[i]) return MOE_FP8_DS_ERR_NULL;
  return run_layer(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
                   gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset,
                   routed_scaling_factor, output, T, workspace, workspace_bytes, stream,
                   stage_events);
}

int moe_fp8_ds_run_noalloc(const float* routing_logits, const void* routing_bias, const void* hidden_states,
                           const float* hidden_states_scale, const void* gemm1_weights,
                           const float* gemm1_weights_scale, const void* gemm2_weights,
                           const float* gemm2_weights_scale, int64_t local_expert_offset,
                           double routed_scaling_factor, void* output, int64_t T, hipStream_t stream) {
  // the order of check_common, so that both entry points return the same
  // status for the same bad argument; the scratch limit comes after them
  if (T < 0 || T > moe::kMaxTokens) return MOE_FP8_DS_ERR_SHAPE;
  if (!std::isfinite(routed_scaling_factor)) return MOE_FP8_DS_ERR_ARG;
  if (T > MOE_FP8_DS_NOALLOC_MAX_TOKENS) return MOE_FP8_DS_ERR_SCRATCH;
  if (T == 0) return MOE_FP8_DS_OK;
  void* ws = noalloc_scratch();
  if (!ws) return MOE_FP8_DS_ERR_HIP;
  // The layer needs no initialised workspace (every region it reads is
  // written earlier in the same call), so nothing is cleared here.
  return run_layer(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
                   gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset,
                   routed_scaling_factor, output, T, ws, kNoAllocScratchBytes, stream, nullptr);
}

int moe_fp8_ds_quantize_hidden(const void* hidden_bf16, int64_t T, void* hidden_fp8, float* hidden_scale,
                               hipStream_t stream) {
  if (T < 0 || T > moe::kMaxTokens) return MOE_FP8_DS_ERR_SHAPE;
  if (T == 0) return MOE_FP8_DS_OK;
  if (!hidden_bf16 || !hidden_fp8 || !hidden_scale) return MOE_FP8_DS_ERR_NULL;
  // the kernel stores e4m3 rows 16 bytes at a time
  if (!aligned16(hidden_bf16) || !aligned16(hidden_fp8) || ((uintptr_t)hidden_scale & 3u))
    return MOE_FP8_DS_ERR_ALIGN;
  const hipError_t err = moe::launch_quantize_hidden((const uint16_t*)hidden_bf16, (int)T, (uint8_t*)hidden_fp8,
                                                     hidden_scale, stream);
  return err == hipSuccess ? MOE_FP8_DS_OK : MOE_FP8_DS_ERR_HIP;
}

}  // extern "C"
