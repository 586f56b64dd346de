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

// 896 threads x 8 columns = one 7168-column row per workgroup; every lane
// issues its (up to 8 rows x 2) 16-byte loads of fp32 GEMM2 rows before the
// first add.  Thread i takes columns 4i .. 4i+3 and 3584 + 4i .. +3, so each
// load instruction of a wave covers 1 KB of contiguous bytes.  The rows are
// read once, with nontemporal loads (at T = 8192: 201 -> 183 us).
constexpr int kCombThreads = 896;
constexpr int kCombHalf = kH / 2;
static_assert(kCombThreads * 4 == kCombHalf, "one row per workgroup");

__global__ void __launch_bounds__(kCombThreads)
combine_kernel(const float* __restrict__ down, const int32_t* __restrict__ pair_row,
               const float* __restrict__ topk_w, uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int c[2] = {(int)threadIdx.x * 4, kCombHalf + (int)threadIdx.x * 4};
  int row[kTopK];
  float w[kTopK];
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    row[k] = pair_row[(size_t)t * kTopK + k];
    w[k] = topk_w[(size_t)t * kTopK + k];
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
  hipLaunchKernelGGL(combine_kernel, dim3(T), dim3(kCombThreads), 0, stream,
                     (const float*)(ws + L.down), (const int32_t*)(ws + L.pair_row),
                     (const float*)(ws + L.topk_w), (uint16_t*)out);
  return hipGetLastError();
}

}  // namespace moe
