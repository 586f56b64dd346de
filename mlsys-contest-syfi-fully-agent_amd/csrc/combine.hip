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

constexpr int kCombThreads = 256;

__global__ void __launch_bounds__(kCombThreads)
combine_kernel(const uint16_t* __restrict__ down, const int32_t* __restrict__ pair_row,
               const float* __restrict__ topk_w, uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  int row[kTopK];
  float w[kTopK];
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    row[k] = pair_row[(size_t)t * kTopK + k];
    w[k] = topk_w[(size_t)t * kTopK + k];
  }
  for (int c = threadIdx.x * 4; c < kH; c += kCombThreads * 4) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int k = 0; k < kTopK; ++k) {
      if (row[k] < 0) continue;
      const uint2 v = *(const uint2*)(down + (size_t)row[k] * kH + c);
      a0 = a0 + bf16_to_f32((uint16_t)v.x) * w[k];
      a1 = a1 + bf16_to_f32((uint16_t)(v.x >> 16)) * w[k];
      a2 = a2 + bf16_to_f32((uint16_t)v.y) * w[k];
      a3 = a3 + bf16_to_f32((uint16_t)(v.y >> 16)) * w[k];
    }
    uint2 packed;
    packed.x = (uint32_t)f32_to_bf16_rne(a0) | ((uint32_t)f32_to_bf16_rne(a1) << 16);
    packed.y = (uint32_t)f32_to_bf16_rne(a2) | ((uint32_t)f32_to_bf16_rne(a3) << 16);
    *(uint2*)(out + (size_t)t * kH + c) = packed;
  }
}

}  // namespace

hipError_t launch_combine(int T, const Layout& L, char* ws, void* out, hipStream_t stream) {
  hipLaunchKernelGGL(combine_kernel, dim3(T), dim3(kCombThreads), 0, stream,
                     (const uint16_t*)(ws + L.down), (const int32_t*)(ws + L.pair_row),
                     (const float*)(ws + L.topk_w), (uint16_t*)out);
  return hipGetLastError();
}

}  // namespace moe
