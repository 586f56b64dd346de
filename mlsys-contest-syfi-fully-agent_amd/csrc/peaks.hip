// peaks.hip -- microbenchmarks for the measured roofline denominators that
// bench.py reports beside MI355X's published peaks (not part of the layer;
// built into lib/libmoe_bench.so):
//   * streaming read: every byte of a buffer read once with 16-byte nontemporal loads
//     (what the layer's HBM-bound kernels do with the expert weights);
//   * MFMA issue rate: independent accumulator chains of the two instructions
//     the GEMMs use (v_mfma_f32_16x16x128_f8f6f4 and v_mfma_f32_16x16x32_bf16),
//     operands in registers, launched by bench.py at 16 waves per CU; once
//     with fixed operands and once with random ones, whose switching power
//     lowers the clock the chip sustains;
//   * trace markers: two empty kernels whose dispatches split a kernel trace
//     of several workloads' calls into per-workload spans.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kChains = 8;

constexpr int kReadUnroll = 8;  // 16-byte loads in flight per lane

// Workgroup b reads the contiguous words [b * chunk, (b + 1) * chunk) of the
// n 16-byte words with nontemporal loads, kReadUnroll per lane in flight
// (chunk = n / gridDim.x, a multiple of 256 * kReadUnroll: the host checks).
// The xor keeps the loads live and is written once per thread.  Measured on
// MI355X against the alternatives: a grid-stride loop reaches 6.2-6.5 TB/s,
// temporal loads 6.2-6.3 TB/s, this 6.7-7.1 TB/s (best at 4 workgroups/CU).
__global__ void __launch_bounds__(256) read_stream(const v4u* __restrict__ src, size_t n, uint32_t* __restrict__ sink) {
  v4u x = {0u, 0u, 0u, 0u};
  const size_t chunk = n / gridDim.x;
  const v4u* p = src + (size_t)blockIdx.x * chunk + threadIdx.x;
  for (size_t j = 0; j < chunk; j += 256 * kReadUnroll) {
    v4u v[kReadUnroll];
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) v[u] = __builtin_nontemporal_load(p + j + u * 256);
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) x ^= v[u];
  }
  sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = x[0] ^ x[1] ^ x[2] ^ x[3];
}

__global__ void __launch_bounds__(512) mfma_f8_loop(int iters, float* __restrict__ sink) {
  const int l = threadIdx.x & 63;
  v8i a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = 0x38383838 ^ (l + i);  // e4m3 values near 1
    b[i] = 0x38383838 ^ (3 * l + i);
  }
  v4f acc[kChains] = {};
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int j = 0; j < kChains; ++j)
      acc[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc[j], 0, 0, 0, 0, 0, 0);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kChains; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

__global__ void __launch_bounds__(512) mfma_bf16_loop(int iters, float* __restrict__ sink) {
  const int l = threadIdx.x & 63;
  v8bf a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(1.0f + (l + i) * 0.0078125f);
    b[i] = (__bf16)(1.0f - (l + 2 * i) * 0.0039062f);
  }
  v4f acc[kChains] = {};
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int j = 0; j < kChains; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[j], 0, 0, 0);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kChains; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Random operands: four register sets per wave from an integer hash of the
// thread and set index, chain j multiplying set j % 4 by set (j + 1) % 4, so
// consecutive MFMAs see different bits, as a GEMM's operands do.  e4m3 bytes
// are masked to 0x77 (finite, |x| < 1.5 * 2^7); bf16 values lie in [-1, 1).
__device__ __forceinline__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x21f0aaadU;
  x ^= x >> 15;
  x *= 0xd35a2d97U;
  x ^= x >> 15;
  return x;
}
constexpr int kSets = 4;

__global__ void __launch_bounds__(512) mfma_f8_loop_random(int iters, float* __restrict__ sink) {
  const uint32_t g = blockIdx.x * 512u + threadIdx.x;
  v8i a[kSets], b[kSets];
#pragma unroll
  for (int j = 0; j < kSets; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[j][i] = (int)(mix32(g * 64u + 8u * j + i) & 0x77777777u);
      b[j][i] = (int)(mix32(g * 64u + 32u + 8u * j + i) & 0x77777777u);
    }
  v4f acc[kChains] = {};
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int j = 0; j < kChains; ++j)
      acc[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[j % kSets], b[(j + 1) % kSets], acc[j], 0, 0, 0,
                                                                 0, 0, 0);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kChains; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  sink[g] = s;
}

__global__ void __launch_bounds__(512) mfma_bf16_loop_random(int iters, float* __restrict__ sink) {
  const uint32_t g = blockIdx.x * 512u + threadIdx.x;
  v8bf a[kSets], b[kSets];
#pragma unroll
  for (int j = 0; j < kSets; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[j][i] = (__bf16)((float)(mix32(g * 64u + 8u * j + i) & 0xFFFFu) * (1.0f / 32768.0f) - 1.0f);
      b[j][i] = (__bf16)((float)(mix32(g * 64u + 32u + 8u * j + i) & 0xFFFFu) * (1.0f / 32768.0f) - 1.0f);
    }
  v4f acc[kChains] = {};
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int j = 0; j < kChains; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j % kSets], b[(j + 1) % kSets], acc[j], 0, 0, 0);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kChains; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  sink[g] = s;
}

__global__ void trace_mark_begin() {}
__global__ void trace_mark_end() {}

}  // namespace

extern "C" {

// Reads `bytes` of `src` once; `bytes` must be a multiple of
// blocks * 256 * 16 * kReadUnroll (else hipErrorInvalidValue, nothing
// launched).  `sink` holds blocks * 256 uint32.  Returns a hipError_t.
int moe_bench_read_stream(const void* src, size_t bytes, void* sink, int blocks, hipStream_t stream) {
  if (blocks <= 0 || bytes % ((size_t)blocks * 256 * 16 * kReadUnroll) != 0) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(read_stream, dim3(blocks), dim3(256), 0, stream, (const v4u*)src, bytes / 16, (uint32_t*)sink);
  return (int)hipGetLastError();
}

// kind 0: fp8 f8f6f4 16x16x128, kind 1: bf16 16x16x32, fixed operands;
// kinds 2 and 3: the same with random operands.  `blocks` workgroups
// of 512 threads, each wave `iters` x 8 MFMAs; `sink` holds blocks * 512
// floats.  FLOPs = blocks * 8 waves * iters * 8 * (2 * 16 * 16 * K).
int moe_bench_mfma_loop(int kind, int iters, int blocks, void* sink, hipStream_t stream) {
  if (kind == 0)
    hipLaunchKernelGGL(mfma_f8_loop, dim3(blocks), dim3(512), 0, stream, iters, (float*)sink);
  else if (kind == 1)
    hipLaunchKernelGGL(mfma_bf16_loop, dim3(blocks), dim3(512), 0, stream, iters, (float*)sink);
  else if (kind == 2)
    hipLaunchKernelGGL(mfma_f8_loop_random, dim3(blocks), dim3(512), 0, stream, iters, (float*)sink);
  else if (kind == 3)
    hipLaunchKernelGGL(mfma_bf16_loop_random, dim3(blocks), dim3(512), 0, stream, iters, (float*)sink);
  else
    return (int)hipErrorInvalidValue;
  return (int)hipGetLastError();
}

// Dispatches the empty kernel trace_mark_begin (end = 0) or trace_mark_end
// (end != 0) on `stream`.  Returns a hipError_t.
int moe_bench_trace_mark(int end, hipStream_t stream) {
  if (end)
    hipLaunchKernelGGL(trace_mark_end, dim3(1), dim3(64), 0, stream);
  else
    hipLaunchKernelGGL(trace_mark_begin, dim3(1), dim3(64), 0, stream);
  return (int)hipGetLastError();
}

}  // extern "C"
