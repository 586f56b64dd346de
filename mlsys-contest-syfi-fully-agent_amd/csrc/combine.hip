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

// 448 threads x 16 columns = one 7168-column row per workgroup; every lane
// issues its (up to 8 rows x 2) 16-byte loads before the first add.  Thread i
// takes the 8-column chunks i and i + 448, so each load or store instruction
// of a wave covers 1 KB of contiguous bytes.
constexpr int kCombThreads = 448;
constexpr int kCombCols = 16;
static_assert(kCombThreads * kCombCols == kH, "one row per workgroup");

__global__ void __launch_bounds__(kCombThreads)
combine_kernel(const uint16_t* __restrict__ down, const int32_t* __restrict__ pair_row,
               const float* __restrict__ topk_w, uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int c0 = threadIdx.x * 8, c1 = (threadIdx.x + kCombThreads) * 8;  // chunk h starts at column c_h
  int row[kTopK];
  float w[kTopK];
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    row[k] = pair_row[(size_t)t * kTopK + k];
    w[k] = topk_w[(size_t)t * kTopK + k];
  }
  uint4 v[kTopK][2];
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    const uint16_t* src = down + (size_t)max(row[k], 0) * kH;
    if (row[k] >= 0) {
      v[k][0] = *(const uint4*)(src + c0);
      v[k][1] = *(const uint4*)(src + c1);
    }
  }
  float a[kCombCols];
#pragma unroll
  for (int i = 0; i < kCombCols; ++i) a[i] = 0.f;
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    if (row[k] < 0) continue;  // token-uniform
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t u[4] = {v[k][h].x, v[k][h].y, v[k][h].z, v[k][h].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        a[8 * h + 2 * q] = a[8 * h + 2 * q] + bf16_to_f32((uint16_t)u[q]) * w[k];
        a[8 * h + 2 * q + 1] = a[8 * h + 2 * q + 1] + bf16_to_f32((uint16_t)(u[q] >> 16)) * w[k];
      }
    }
  }
  uint4 o[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t p[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      p[q] = (uint32_t)f32_to_bf16_rne(a[8 * h + 2 * q]) | ((uint32_t)f32_to_bf16_rne(a[8 * h + 2 * q + 1]) << 16);
    o[h] = uint4{p[0], p[1], p[2], p[3]};
  }
  *(uint4*)(out + (size_t)t * kH + c0) = o[0];
  *(uint4*)(out + (size_t)t * kH + c1) = o[1];
}

}  // namespace

hipError_t launch_combine(int T, const Layout& L, char* ws, void* out, hipStream_t stream) {
  hipLaunchKernelGGL(combine_kernel, dim3(T), dim3(kCombThreads), 0, stream,
                     (const uint16_t*)(ws + L.down), (const int32_t*)(ws + L.pair_row),
                     (const float*)(ws + L.topk_w), (uint16_t*)out);
  return hipGetLastError();
}

}  // namespace moe
