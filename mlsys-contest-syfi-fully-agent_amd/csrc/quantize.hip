// quantize.hip -- the step before the layer: bf16 hidden states -> e4m3 rows
// with one fp32 scale per 128-column block, stored transposed ([56, T]), i.e.
// exactly the `hidden_states` / `hidden_states_scale` pair the layer consumes
// (layout: moe.py:32-33; the reference repository holds no quantiser, so the
// convention is the DeepSeek-V3 one this build's generator also uses):
//   scale = absmax(block) / 448          (1 for an all-zero block)
//   q     = e4m3(x / scale), round to nearest even, saturating to +-448
// NaN elements do not enter the absmax and encode as NaN.
//
// Design (gfx950): HBM-bound (reads 2 B and writes 1 B per element).  One
// wave per token row; each pass of a wave covers 512 columns = 4 scale blocks
// with 16 lanes per block, every lane loading 16 contiguous bytes (8 bf16).
// A block's absmax is a 16-lane max; the wave's scales go through LDS so that
// the transposed scale rows are written as 16 contiguous tokens.
#include "kernels.hpp"

namespace moe {
namespace {

constexpr int kQTokens = 16;  // tokens (waves) per workgroup
constexpr int kQThreads = kQTokens * kWave;
constexpr int kQPass = 512;   // columns per wave pass

// fp32 -> OCP e4m3fn, round to nearest even, saturating finite values;
// NaN -> 0x7F (sign kept).
__device__ __forceinline__ uint32_t f32_to_e4m3_satfinite(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7Fu;
  const float af = __uint_as_float(a);
  if (af >= 448.0f) return sign | 0x7Eu;
  if (af < 0x1p-6f) return sign | (uint32_t)rintf(af * 512.0f);  // subnormal grid 2^-9, RNE
  int e = (int)(a >> 23) - 127;
  uint32_t keep = (a >> 20) & 7u;
  const uint32_t rem = a & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (keep & 1u))) {
    if (++keep == 8u) {
      keep = 0;
      ++e;
    }
  }
  if (e > 8 || (e == 8 && keep == 7u)) return sign | 0x7Eu;
  return sign | ((uint32_t)(e + 7) << 3) | keep;
}

__device__ __forceinline__ float fmax_nonnan(float a, float b) { return b > a ? b : a; }

__global__ void __launch_bounds__(kQThreads)
quantize_hidden_kernel(const uint16_t* __restrict__ x, int T, uint8_t* __restrict__ q,
                       float* __restrict__ scale) {
  __shared__ float sc[kNHBlk][kQTokens];
  const int w = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int t = blockIdx.x * kQTokens + w;
  if (t < T) {
    const uint16_t* row = x + (size_t)t * kH;
    uint8_t* qrow = q + (size_t)t * kH;
#pragma unroll 2
    for (int c = 0; c < kH / kQPass; ++c) {
      const int col = c * kQPass + lane * 8;
      const uint4 raw = *(const uint4*)(row + col);
      const uint32_t u[4] = {raw.x, raw.y, raw.z, raw.w};
      float v[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(u[i] << 16);
        v[2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
      }
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmax_nonnan(amax, fabsf(v[i]));
      // max over the 16 lanes of this block (xor 1, 2, 4, 8 stay inside it)
#pragma unroll
      for (int m = 1; m < 16; m <<= 1) amax = fmax_nonnan(amax, __shfl_xor(amax, m, kWave));
      const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lo |= f32_to_e4m3_satfinite(v[i] / s) << (8 * i);
        hi |= f32_to_e4m3_satfinite(v[4 + i] / s) << (8 * i);
      }
      *(uint2*)(qrow + col) = uint2{lo, hi};
      if ((lane & 15) == 0) sc[c * 4 + (lane >> 4)][w] = s;
    }
  }
  __syncthreads();
  // scale[b][t0 .. t0+15]: 16 contiguous floats per block row
  const int t0 = blockIdx.x * kQTokens;
  for (int i = threadIdx.x; i < kNHBlk * kQTokens; i += kQThreads) {
    const int b = i / kQTokens, k = i % kQTokens;
    if (t0 + k < T) scale[(size_t)b * T + t0 + k] = sc[b][k];
  }
}

}  // namespace

hipError_t launch_quantize_hidden(const uint16_t* x, int T, uint8_t* q, float* scale, hipStream_t stream) {
  const int blocks = (T + kQTokens - 1) / kQTokens;
  hipLaunchKernelGGL(quantize_hidden_kernel, dim3(blocks), dim3(kQThreads), 0, stream, x, T, q, scale);
  return hipGetLastError();
}

}  // namespace moe
