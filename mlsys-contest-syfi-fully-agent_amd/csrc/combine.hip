// combine.hip -- routing-weighted combine of the GEMM2 rows into the bf16
// output.
//
// Reference behaviour: moe.py:163 (zero fp32 accumulator), moe.py:199-200
// (output.index_add_(token, O * w), experts in ascending order) and moe.py:202
// (.to(bfloat16)); CUDA solution: fp32 atomicAdd in the GEMM2 epilogue
// (moe.cu:2404-2430) plus memset and fin_cast8_kernel (moe.cu:2473-2496).
//
// Here each token gathers its (at most 8) local rows in ascending expert order
// and forms  acc = acc + (O * w)  with two separately rounded fp32 ops, exactly
// the reference's accumulation order, with no atomics, no memset and a
// deterministic result.  Every output element is written (tokens without a
// local expert get zeros).
#include "moe_common.hpp"

namespace moe {
namespace {

// A workgroup of kCombThreads threads combines kCombCols columns of one
// token: thread i takes columns 4i .. 4i+3 and kCombCols / 2 + 4i .. +3 of
// its part, so each load instruction of a wave covers 1 KB of contiguous
// bytes, and every lane issues its (up to 8 rows x 2) 16-byte loads of fp32
// GEMM2 rows before the first add.  The rows are read once, with
// nontemporal loads (at T = 8192: 201 -> 183 us).  One wave per workgroup,
// 14 per token: many small workgroups per CU overlap their index loads with
// other tokens' row loads (interleaved runs, T = 4096 / 8192 / 14107: 93.2 /
// 183.3 / 318.7 us with one 896-thread workgroup per token, 89.9 / 179.0 /
// 311.5 with 64 threads; 448 and 128 threads in between; same bits).
constexpr int kCombThreads = 64;
constexpr int kCombCols = 8 * kCombThreads;
constexpr int kCombParts = kH / kCombCols;  // workgroups per token
static_assert(kCombParts * kCombCols == kH && kCombThreads % kWave == 0, "whole waves, whole parts");

__global__ void __launch_bounds__(kCombThreads)
combine_kernel(const float* __restrict__ down, const int32_t* __restrict__ pair_row,
               const float* __restrict__ topk_w, const int32_t* __restrict__ expert_off, int T,
               uint16_t* __restrict__ out) {
  const int t = blockIdx.x / kCombParts;
  const int c0 = (blockIdx.x % kCombParts) * kCombCols + (int)threadIdx.x * 4;
  const int c[2] = {c0, c0 + kCombCols / 2};
  int row[kTopK];
  float w[kTopK];
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    row[k] = pair_row[(size_t)t * kTopK + k];
    w[k] = topk_w[(size_t)t * kTopK + k];
  }
  // Experts of every token (every_token_experts): GEMM2 wrote the token's
  // weighted sum over them to the first one's row; add that row once, with
  // weight 1, at its place in expert order, and skip the others' rows.  The
  // row loads wait for this test (the offsets' read costs the pass ~0.4 us
  // at T = 1024), so below the size where it can hold they are not read.
  ExpertRows X;
  uint32_t fused = 0u;
  if (T >= kEveryTokenFuseMinTokens) {  // kernel-uniform
    X.load(expert_off);
    fused = every_token_experts(X, T);
  }
  if (fused) {
#pragma unroll
    for (int k = 0; k < kTopK; ++k) {
      if (row[k] < 0) continue;  // token-uniform
      const int e = expert_of_row(X, row[k]);
      if ((fused >> e) & 1u) {
        if (e == __builtin_ctz(fused))
          w[k] = 1.0f;
        else
          row[k] = -1;
      }
    }
  }
  v4f v[kTopK][2];
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    const float* src = down + (size_t)max(row[k], 0) * kH;
    if (row[k] >= 0) {
      v[k][0] = __builtin_nontemporal_load((const v4f*)(src + c[0]));
      v[k][1] = __builtin_nontemporal_load((const v4f*)(src + c[1]));
    }
  }
  // ascending expert order, acc = acc + (O * w): two roundings, as index_add_
  // of O * w in moe.py:199-200
  float a[2][4] = {};
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    if (row[k] < 0) continue;  // token-uniform
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) a[h][i] = a[h][i] + v[k][h][i] * w[k];
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint2 o{(uint32_t)f32_to_bf16_rne(a[h][0]) | ((uint32_t)f32_to_bf16_rne(a[h][1]) << 16),
                  (uint32_t)f32_to_bf16_rne(a[h][2]) | ((uint32_t)f32_to_bf16_rne(a[h][3]) << 16)};
    *(uint2*)(out + (size_t)t * kH + c[h]) = o;
  }
}

}  // namespace

hipError_t launch_combine(int T, const Layout& L, char* ws, void* out, hipStream_t stream) {
  hipLaunchKernelGGL(combine_kernel, dim3(T * kCombParts), dim3(kCombThreads), 0, stream,
                     (const float*)(ws + L.down), (const int32_t*)(ws + L.pair_row),
                     (const float*)(ws + L.topk_w), (const int32_t*)(ws + L.expert_off), T, (uint16_t*)out);
  return hipGetLastError();
}

}  // namespace moe
