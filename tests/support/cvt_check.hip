// Exhaustive checks of two gfx950 conversion instructions the kernels use.
// (1) The fp32 -> e4m3 conversion instruction that the
// activation quantiser's fast path uses (v_cvt_pk_fp8_f32 through
// __builtin_amdgcn_cvt_pk_fp8_f32), against the software round-to-nearest-even
// conversion of the quantiser's exact path, over all 2^32 fp32 bit patterns.
//
// (2) v_cvt_pk_bf16_f32 (the SwiGLU epilogues' bf16 hi/lo split) against
// software round-to-nearest-even, all 2^32 patterns (bf16_check).
//
// TEST SUPPORT ONLY (tests/test_gpu_quantize.py, tests/test_gpu_mfma_precision.py).  Mismatches are counted by
// the magnitude of the input: [0] |y| <= 448, [1] 448 < |y| < 464,
// [2] |y| >= 464 finite, [3] infinity, [4] NaN; [5] counts lanes whose packed
// result does not have the documented byte layout (src0 -> byte 0, src1 ->
// byte 1; word_sel writes bytes 2-3 and keeps bytes 0-1 of `old`).  The fast
// path only converts |y| <= 448 * (1 + 2^-22), so [0], [1] and [5] must be 0.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

__device__ uint32_t sw_e4m3(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  const uint32_t normal = min(((a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20) - 960u, 0x7Eu);
  const uint32_t sub = (uint32_t)rintf(__uint_as_float(a) * 512.0f);
  uint32_t code = a < 0x3C800000u ? sub : normal;
  code = a > 0x7F800000u ? 0x7Fu : code;
  return sign | code;
}

constexpr int kPerThread = 256;
constexpr int kThreads = 256;
constexpr int kBlocks = (int)((1ull << 32) / ((uint64_t)kPerThread * kThreads));  // 65536

__global__ void __launch_bounds__(kThreads) cvt_check_kernel(unsigned long long* cnt) {
  const uint64_t tid = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  const uint32_t base = (uint32_t)(tid * kPerThread);
  unsigned long long c[6] = {0, 0, 0, 0, 0, 0};
  for (int j = 0; j < kPerThread; j += 2) {
    const uint32_t ii[2] = {base + j, base + j + 1};
    const float x0 = __uint_as_float(ii[0]), x1 = __uint_as_float(ii[1]);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x0, x1, 0, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x0, x1, 0x5A5A, true);
    const uint32_t hw[2] = {lo & 0xFFu, (lo >> 8) & 0xFFu};
    for (int k = 0; k < 2; ++k) {
      if (hw[k] != sw_e4m3(__uint_as_float(ii[k]))) {
        const uint32_t a = ii[k] & 0x7FFFFFFFu;
        ++c[a > 0x7F800000u ? 4 : a == 0x7F800000u ? 3 : a >= 0x43E80000u ? 2 : a > 0x43E00000u ? 1 : 0];
      }
    }
    if ((hi & 0xFFFFu) != 0x5A5Au || (hi >> 16) != (lo & 0xFFFFu) || (lo >> 16) != 0u) ++c[5];
  }
  for (int k = 0; k < 6; ++k)
    if (c[k]) atomicAdd(&cnt[k], c[k]);
}

// fp32 -> bf16 round to nearest even in software (the layer's
// f32_to_bf16_rne, moe_common.hpp).
__device__ uint32_t sw_bf16(uint32_t u) {
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0xFFFFFFFFu;  // NaN: compared separately
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// v_cvt_pk_bf16_f32 (what __builtin_convertvector to a bf16 pair compiles to
// on gfx950) against sw_bf16 for every fp32 pattern; [0] finite or infinite
// mismatches, [1] NaN inputs not giving a NaN, [2] element order of the pair.
__global__ void __launch_bounds__(kThreads) bf16_check_kernel(unsigned long long* cnt) {
  const uint64_t tid = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  const uint32_t base = (uint32_t)(tid * kPerThread);
  unsigned long long c[3] = {0, 0, 0};
  for (int j = 0; j < kPerThread; j += 2) {
    const uint32_t ii[2] = {base + j, base + j + 1};
    const v2bf r = __builtin_convertvector(v2f{__uint_as_float(ii[0]), __uint_as_float(ii[1])}, v2bf);
    const uint32_t p = __builtin_bit_cast(uint32_t, r);
    const uint32_t hw[2] = {p & 0xFFFFu, p >> 16};
    for (int k = 0; k < 2; ++k) {
      const uint32_t sw = sw_bf16(ii[k]);
      if (sw == 0xFFFFFFFFu) {
        if ((hw[k] & 0x7FFFu) <= 0x7F80u) ++c[1];
      } else if (hw[k] != sw) {
        ++c[0];
      }
    }
    const v2bf o = __builtin_convertvector(v2f{1.0f, 2.0f}, v2bf);  // element 0 -> bits 0-15
    if (__builtin_bit_cast(uint32_t, o) != 0x40003F80u) ++c[2];
  }
  for (int k = 0; k < 3; ++k)
    if (c[k]) atomicAdd(&cnt[k], c[k]);
}

}  // namespace

// counts: host array of 3; returns 0 on success, else the HIP error code.
extern "C" int bf16_check(unsigned long long* counts) {
  unsigned long long* d = nullptr;
  hipError_t e = hipMalloc(&d, 3 * sizeof(unsigned long long));
  if (e != hipSuccess) return (int)e;
  e = hipMemset(d, 0, 3 * sizeof(unsigned long long));
  if (e == hipSuccess) {
    hipLaunchKernelGGL(bf16_check_kernel, dim3(kBlocks), dim3(kThreads), 0, 0, d);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(counts, d, 3 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  (void)hipFree(d);
  return (int)e;
}

// counts: host array of 6; returns 0 on success, else the HIP error code.
extern "C" int cvt_check(unsigned long long* counts) {
  unsigned long long* d = nullptr;
  hipError_t e = hipMalloc(&d, 6 * sizeof(unsigned long long));
  if (e != hipSuccess) return (int)e;
  e = hipMemset(d, 0, 6 * sizeof(unsigned long long));
  if (e == hipSuccess) {
    hipLaunchKernelGGL(cvt_check_kernel, dim3(kBlocks), dim3(kThreads), 0, 0, d);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(counts, d, 6 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  (void)hipFree(d);
  return (int)e;
}
