// synth.hip -- deterministic synthetic workload generator on the GPU
// (libmoe_synth.so, declared in include/moe_synth.h).
//
// Stands in for the harness's input generation (flashinfer-bench gen_inputs /
// load_safetensors, called at full-agent-pipeline/scripts/seed_ref_cache.py:78-81),
// which is not available offline.  The definition is integer hashing plus
// IEEE-exact fp32 multiply/divide and integer-coded rounding, so the CPU
// restatement used by the tests produces identical bytes:
//   h      = splitmix64 output at position idx of the stream keyed by
//            mix64((seed << 8) ^ stream)
//   normal = (sum of the four 16-bit fields of h - 131070) * (1/37837.227)
//            (Irwin-Hall(4): approximately N(0,1), bounded at +-3.46)
//   blocks = absmax/448 scale, e4m3 = RNE(x / scale) saturated to +-448.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/moe_synth.h"

namespace {

constexpr int kH = 7168, kI = 2048, k2I = 4096, kE = 32, kEG = 256, kB = 128;
constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;
constexpr float kInvStd = 0x1.bb67aep-16f;
constexpr float kSigmaW13 = 0x1.83091ep-7f;
constexpr float kSigmaW2 = 0x1.6a09e6p-6f;
constexpr float kSigmaBias = 0x1.99999ap-4f;
enum { kLogits = 1, kBias = 2, kHidden = 3, kW13 = 4, kW2 = 5 };

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += kGamma;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ float normal_at(uint64_t key, uint64_t idx) {
  const uint64_t h = mix64(key + idx * kGamma);
  const int32_t s = (int32_t)((h & 0xFFFF) + ((h >> 16) & 0xFFFF) + ((h >> 32) & 0xFFFF) + (h >> 48));
  return (float)(s - 131070) * kInvStd;
}

// fp32 -> OCP e4m3fn, round to nearest even, saturating finite values.
__device__ __forceinline__ uint8_t to_e4m3(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint8_t)(sign | 0x7F);
  const float af = __uint_as_float(a);
  if (af >= 448.0f) return (uint8_t)(sign | 0x7E);
  if (af < 0x1p-6f) return (uint8_t)(sign | (uint8_t)rintf(af * 512.0f));
  int e = (int)(a >> 23) - 127;
  uint32_t keep = (a >> 20) & 7u;
  const uint32_t rem = a & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (keep & 1u))) {
    if (++keep == 8u) {
      keep = 0;
      ++e;
    }
  }
  if (e > 8 || (e == 8 && keep == 7u)) return (uint8_t)(sign | 0x7E);
  return (uint8_t)(sign | (uint8_t)((e + 7) << 3) | (uint8_t)keep);
}

__device__ __forceinline__ uint16_t to_bf16(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float block_scale(float amax) { return amax > 0.0f ? amax / 448.0f : 1.0f; }

__global__ void logits_kernel(uint64_t key, int64_t n, float* __restrict__ out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = normal_at(key, (uint64_t)i);
}

__global__ void bias_kernel(uint64_t key, int n_hot, int32_t h0, int32_t h1, int32_t h2, int32_t h3,
                            int32_t h4, int32_t h5, int32_t h6, int32_t h7, float hot_add,
                            uint16_t* __restrict__ out) {
  const int e = threadIdx.x;
  float b = normal_at(key, (uint64_t)e) * kSigmaBias;
  const int32_t hot[8] = {h0, h1, h2, h3, h4, h5, h6, h7};
  for (int j = 0; j < n_hot; ++j)
    if (hot[j] == e) b = b + hot_add;
  out[e] = to_bf16(b);
}

// One wave per (token, 128-column block).
__global__ void hidden_kernel(uint64_t key, int64_t T, uint8_t* __restrict__ q, float* __restrict__ scale) {
  const int64_t blk = blockIdx.x * (int64_t)(blockDim.x / 64) + threadIdx.x / 64;
  const int lane = threadIdx.x & 63;
  if (blk >= T * (kH / kB)) return;
  const int64_t t = blk / (kH / kB);
  const int b = (int)(blk % (kH / kB));
  const uint64_t idx = (uint64_t)t * kH + (uint64_t)b * kB + 2 * lane;
  const float v0 = normal_at(key, idx), v1 = normal_at(key, idx + 1);
  float amax = fmaxf(fabsf(v0), fabsf(v1));
  for (int m = 1; m < 64; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
  const float s = block_scale(amax);
  if (lane == 0) scale[(int64_t)b * T + t] = s;
  uint8_t* dst = q + t * kH + b * kB + 2 * lane;
  dst[0] = to_e4m3(v0 / s);
  dst[1] = to_e4m3(v1 / s);
}

// One 256-thread block per 128x128 weight block; thread = (row, 64 columns).
__global__ void __launch_bounds__(256) weight_kernel(uint64_t key, float sigma, int rows, int cols, int e0,
                                                     uint8_t* __restrict__ q, float* __restrict__ scale) {
  const int rb_n = rows / kB, cb_n = cols / kB;
  const int64_t bi = blockIdx.x;
  const int e = e0 + (int)(bi / (rb_n * cb_n));
  const int rb = (int)((bi / cb_n) % rb_n);
  const int cb = (int)(bi % cb_n);
  const int r = threadIdx.x >> 1;
  const int c0 = (threadIdx.x & 1) * 64;
  const uint64_t row = (uint64_t)e * rows + (uint64_t)rb * kB + r;
  const uint64_t base = row * (uint64_t)cols + (uint64_t)cb * kB + c0;
  float v[64];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 64; ++j) {
    v[j] = normal_at(key, base + j) * sigma;
    amax = fmaxf(amax, fabsf(v[j]));
  }
  for (int m = 1; m < 64; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
  __shared__ float wmax[4];
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const float s = block_scale(amax);
  if (threadIdx.x == 0) scale[((int64_t)e * rb_n + rb) * cb_n + cb] = s;
  uint8_t* dst = q + row * (uint64_t)cols + (uint64_t)cb * kB + c0;
#pragma unroll
  for (int j = 0; j < 64; j += 16) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      w[k] = (uint32_t)to_e4m3(v[j + 4 * k] / s) | ((uint32_t)to_e4m3(v[j + 4 * k + 1] / s) << 8) |
             ((uint32_t)to_e4m3(v[j + 4 * k + 2] / s) << 16) | ((uint32_t)to_e4m3(v[j + 4 * k + 3] / s) << 24);
    *(uint4*)(dst + j) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

int status(hipError_t e) { return e == hipSuccess ? 0 : -5; }

}  // namespace

extern "C" {

int moe_synth_logits(uint64_t seed, int64_t T, float* out, hipStream_t stream) {
  if (T < 0) return -2;
  if (T == 0) return 0;
  if (!out) return -1;
  const int64_t n = T * kEG;
  const int blocks = (int)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536);
  hipLaunchKernelGGL(logits_kernel, dim3(blocks), dim3(256), 0, stream, mix64((seed << 8) ^ kLogits), n, out);
  return status(hipGetLastError());
}

int moe_synth_bias(uint64_t seed, const int32_t* hot_ids, int n_hot, float hot_add, uint16_t* out,
                   hipStream_t stream) {
  if (!out || (n_hot > 0 && !hot_ids)) return -1;
  if (n_hot < 0 || n_hot > 8) return -6;
  int32_t h[8] = {-1, -1, -1, -1, -1, -1, -1, -1};
  for (int j = 0; j < n_hot; ++j) h[j] = hot_ids[j];
  hipLaunchKernelGGL(bias_kernel, dim3(1), dim3(kEG), 0, stream, mix64((seed << 8) ^ kBias), n_hot, h[0],
                     h[1], h[2], h[3], h[4], h[5], h[6], h[7], hot_add, out);
  return status(hipGetLastError());
}

int moe_synth_hidden(uint64_t seed, int64_t T, uint8_t* q, float* scale, hipStream_t stream) {
  if (T < 0) return -2;
  if (T == 0) return 0;
  if (!q || !scale) return -1;
  const int64_t nblk = T * (kH / kB);
  hipLaunchKernelGGL(hidden_kernel, dim3((unsigned)((nblk + 3) / 4)), dim3(256), 0, stream,
                     mix64((seed << 8) ^ kHidden), T, q, scale);
  return status(hipGetLastError());
}

static int weight(uint64_t seed, int stream_id, float sigma, int rows, int cols, int e0, int e1, uint8_t* q,
                  float* scale, hipStream_t stream) {
  if (!q || !scale) return -1;
  if (e0 < 0 || e1 > kE || e0 > e1) return -2;
  if (e0 == e1) return 0;
  const int64_t nblk = (int64_t)(e1 - e0) * (rows / kB) * (cols / kB);
  hipLaunchKernelGGL(weight_kernel, dim3((unsigned)nblk), dim3(256), 0, stream,
                     mix64((seed << 8) ^ (uint64_t)stream_id), sigma, rows, cols, e0, q, scale);
  return status(hipGetLastError());
}

int moe_synth_w13(uint64_t seed, int e0, int e1, uint8_t* q, float* scale, hipStream_t stream) {
  return weight(seed, kW13, kSigmaW13, k2I, kH, e0, e1, q, scale, stream);
}

int moe_synth_w2(uint64_t seed, int e0, int e1, uint8_t* q, float* scale, hipStream_t stream) {
  return weight(seed, kW2, kSigmaW2, kH, kI, e0, e1, q, scale, stream);
}

}  // extern "C"
