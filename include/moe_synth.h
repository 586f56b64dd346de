/*
 * moe_synth.h -- deterministic synthetic inputs for the FP8 MoE layer
 * (libmoe_synth.so), generated on the GPU directly into device memory.
 *
 * Stands in for the benchmark harness's input generation (flashinfer-bench
 * gen_inputs / load_safetensors, called from
 * full-agent-pipeline/scripts/seed_ref_cache.py:78-81), which is unavailable
 * offline.  Output layouts are those of include/moe_fp8_ds.h.  The byte stream
 * is fixed by (seed, tensor) and is identical to the CPU generator the tests
 * use.  Returns 0 on success, -1 null pointer, -2 bad size/range, -5 HIP
 * launch failure, -6 bad argument.  All calls are stream-ordered.
 */
#ifndef MOE_SYNTH_H
#define MOE_SYNTH_H

#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* routing_logits [T,256] fp32 ~N(0,1); row t depends only on (seed, t). */
int moe_synth_logits(uint64_t seed, int64_t T, float* out, hipStream_t stream);
/* routing_bias [256] bf16 ~N(0,0.1), plus hot_add on up to 8 expert ids
 * (hot_ids is a host array). */
int moe_synth_bias(uint64_t seed, const int32_t* hot_ids, int n_hot, float hot_add, uint16_t* out,
                   hipStream_t stream);
/* hidden_states [T,7168] e4m3 and hidden_states_scale [56,T] (absmax/448). */
int moe_synth_hidden(uint64_t seed, int64_t T, uint8_t* q, float* scale, hipStream_t stream);
/* gemm1 weights [32,4096,7168] e4m3 ~N(0,1/sqrt(7168)) and [32,32,56] block
 * scales; fills experts [e0, e1) only. */
int moe_synth_w13(uint64_t seed, int e0, int e1, uint8_t* q, float* scale, hipStream_t stream);
/* gemm2 weights [32,7168,2048] e4m3 ~N(0,1/sqrt(2048)) and [32,56,16] block
 * scales; fills experts [e0, e1) only. */
int moe_synth_w2(uint64_t seed, int e0, int e1, uint8_t* q, float* scale, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
