// Accumulation precision of the two MFMA instructions the layer's GEMMs use,
// on caller-supplied operands (TEST SUPPORT ONLY, tests/test_gpu_mfma_precision.py):
//   kind 0: v_mfma_f32_16x16x128_f8f6f4, e4m3 x e4m3, one instruction per
//           16 x 16 x 128 tile (GEMM1: one 128-wide scale block per MFMA);
//   kind 1: v_mfma_f32_16x16x32_bf16, four chained instructions per
//           16 x 16 x 128 tile (GEMM2: fp32 accumulation across K).
// A tile: 16 rows x 128 K; B tile: 16 columns x 128 K (row n of B^T); the
// caller compares D with exact sums.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// one wave per tile; lane (q, r) supplies K bytes 32q .. 32q+31 of row r
__global__ void tile_f8(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B, float* __restrict__ D) {
  const int t = blockIdx.x, l = threadIdx.x, q = l >> 4, r = l & 15;
  const v8i a = *(const v8i*)(A + ((size_t)t * 16 + r) * 128 + 32 * q);
  const v8i b = *(const v8i*)(B + ((size_t)t * 16 + r) * 128 + 32 * q);
  const v4f z = {0.f, 0.f, 0.f, 0.f};
  const v4f d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 0, 0, 0);
  for (int i = 0; i < 4; ++i) D[((size_t)t * 16 + 4 * q + i) * 16 + r] = d[i];
}

// lane (q, r) supplies K values 32s + 8q .. +7 of row r to instruction s
__global__ void tile_bf16(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, float* __restrict__ D) {
  const int t = blockIdx.x, l = threadIdx.x, q = l >> 4, r = l & 15;
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < 4; ++s) {
    const v8bf a = *(const v8bf*)(A + ((size_t)t * 16 + r) * 128 + 32 * s + 8 * q);
    const v8bf b = *(const v8bf*)(B + ((size_t)t * 16 + r) * 128 + 32 * s + 8 * q);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  for (int i = 0; i < 4; ++i) D[((size_t)t * 16 + 4 * q + i) * 16 + r] = acc[i];
}

}  // namespace

// n tiles; A, B host arrays of n * 16 * 128 elements (bytes for kind 0, bf16
// bits for kind 1); D host array of n * 256 floats.  Returns 0 on success.
extern "C" int mfma_tiles(int kind, int n, const void* A, const void* B, float* D) {
  if (n <= 0 || (kind != 0 && kind != 1)) return -1;
  const size_t elem = kind == 0 ? 1 : 2, in_bytes = (size_t)n * 16 * 128 * elem, out_bytes = (size_t)n * 256 * 4;
  void *dA = nullptr, *dB = nullptr, *dD = nullptr;
  int rc = -2;
  if (hipMalloc(&dA, in_bytes) == hipSuccess && hipMalloc(&dB, in_bytes) == hipSuccess &&
      hipMalloc(&dD, out_bytes) == hipSuccess && hipMemcpy(dA, A, in_bytes, hipMemcpyHostToDevice) == hipSuccess &&
      hipMemcpy(dB, B, in_bytes, hipMemcpyHostToDevice) == hipSuccess) {
    if (kind == 0)
      hipLaunchKernelGGL(tile_f8, dim3(n), dim3(64), 0, 0, (const uint8_t*)dA, (const uint8_t*)dB, (float*)dD);
    else
      hipLaunchKernelGGL(tile_bf16, dim3(n), dim3(64), 0, 0, (const uint16_t*)dA, (const uint16_t*)dB, (float*)dD);
    if (hipGetLastError() == hipSuccess && hipMemcpy(D, dD, out_bytes, hipMemcpyDeviceToHost) == hipSuccess) rc = 0;
  }
  (void)hipFree(dA);
  (void)hipFree(dB);
  (void)hipFree(dD);
  return rc;
}
