// quantize.hip -- the step before the layer: bf16 hidden states -> e4m3 rows
// with one fp32 scale per 128-column block, stored transposed ([56, T]), i.e.
// exactly the `hidden_states` / `hidden_states_scale` pair the layer consumes
// (layout: moe.py:32-33; the reference repository holds no quantiser, so the
// convention is the DeepSeek-V3 one this build's generator also uses):
//   scale = absmax(block) / 448          (1 for an all-zero block)
//   q     = e4m3(x / scale), round to nearest even, saturating to +-448
// NaN elements do not enter the absmax and encode as NaN.
//
// Design (gfx950): HBM-bound (reads 2 B and writes 1 B per element), so the
// arithmetic per element has to stay under the memory time.  Up to T = 2048
// one workgroup per token row, wave p quantising pass p (7 waves per row, so
// that enough loads are in flight at small T).  Beyond, one wave per token
// row, four rows per workgroup (T/4 workgroups: 2048 at T = 8192).  A
// wave issues all 14 row loads (16 B per lane each) before any arithmetic, so
// a token has its whole 14 KB row in flight at once; each of the 7 passes
// then covers 1024 columns = 8 scale blocks, 8 lanes per block and 16
// contiguous elements per lane.  A block's absmax is an 8-lane DPP max of
// bf16 magnitudes (compared as integers); the scales go through LDS so that
// each transposed scale row is written as 4 contiguous tokens.
//
// Fast path (every pass whose blocks all have 2^-96 <= absmax < inf or
// absmax = 0, and no NaN): with s = absmax / 448 and r = 1 / s (both
// correctly rounded),
//   q = x * r;  q' = fma(fma(-s, q, x), r, q);  code = e4m3_rne(|q'|) | sign(x)
// and the rounding to e4m3 is v_cvt_pk_fp8_f32.  Both steps were checked
// exhaustively against the correctly rounded x / s followed by the software
// RNE conversion below: q' gives the same e4m3 code for every bf16 pair
// |x| <= absmax in that range (about 1.07e9 pairs), and the hardware
// conversion equals the software one for every fp32 with |y| < 464 (|q'| is
// at most 448 * (1 + 2^-22)).  Passes with a NaN, an infinity or a tiny
// absmax in any of the wave's blocks take the exact path (IEEE division and
// the software conversion) instead; that branch is wave-uniform.
#include "kernels.hpp"

namespace moe {
namespace {

constexpr int kQTokens = 4;   // tokens (waves) per workgroup
constexpr int kQThreads = kQTokens * kWave;
constexpr int kQLaneCols = 16;                 // elements per lane per pass
constexpr int kQPass = kWave * kQLaneCols;     // 1024 columns per wave pass
constexpr int kQPasses = kH / kQPass;          // 7
constexpr int kQLanesPerBlk = kBlk / kQLaneCols;  // 8
constexpr uint32_t kQTinyBf16 = 0x0F80u;       // bf16 bits of 2^-96

// fp32 -> OCP e4m3fn, round to nearest even, saturating finite values and
// infinities to +-448; NaN -> 0x7F (sign kept).  Branch-free:
//   normal range (|x| >= 2^-6): adding 2^19 - 1 + (bit 20) to the magnitude's
//     bits rounds its 23-bit mantissa to 3 bits, nearest even, with the carry
//     running into the exponent; the code is then (bits >> 20) - (120 << 3)
//     (exponent rebias 127 -> 7), clamped to 0x7E (448);
//   subnormal range: the code is |x| / 2^-9 rounded to nearest even (0..8,
//     8 being the smallest normal, 0x08).
__device__ __forceinline__ uint32_t f32_to_e4m3_satfinite(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  const uint32_t normal = min(((a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20) - 960u, 0x7Eu);
  const uint32_t sub = (uint32_t)rintf(__uint_as_float(a) * 512.0f);
  uint32_t code = a < 0x3C800000u ? sub : normal;
  code = a > 0x7F800000u ? 0x7Fu : code;
  return sign | code;
}

__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xFFFF0000u); }

// Largest bf16 magnitude (as bits, 0..0x7FFF) of the 16 elements of one lane;
// NaN patterns (> 0x7F80) order above every number, so a NaN shows as > 0x7F80.
__device__ __forceinline__ uint32_t lane_absmax_bits(const uint4& a, const uint4& b) {
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    lo = max(lo, w[i] & 0x7FFFu);
    hi = max(hi, (w[i] >> 16) & 0x7FFFu);
  }
  return max(lo, hi);
}

// The same with NaN elements left out (the exact path's absmax).
__device__ __forceinline__ uint32_t lane_absmax_bits_nonnan(const uint4& a, const uint4& b) {
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t lo = w[i] & 0x7FFFu, hi = (w[i] >> 16) & 0x7FFFu;
    m = max(m, lo > 0x7F80u ? 0u : lo);
    m = max(m, hi > 0x7F80u ? 0u : hi);
  }
  return m;
}

// Maximum over each group of 8 lanes (a scale block), in every lane of it.
__device__ __forceinline__ uint32_t group8_max_u32(uint32_t k) {
  k = max(k, dpp_u32<kDppQuad1032, 0xF>(k));
  k = max(k, dpp_u32<kDppQuad2301, 0xF>(k));
  return max(k, dpp_u32<kDppRowHalfMirror, 0xF>(k));
}

// Four elements (signs from the inputs) -> four e4m3 bytes, fast path.
__device__ __forceinline__ uint32_t fast_pack4(float x0, float x1, float x2, float x3, float s, float r) {
  const float x[4] = {x0, x1, x2, x3};
  float y[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float q = x[i] * r;
    const float q2 = fmaf(fmaf(-s, q, x[i]), r, q);
    y[i] = __uint_as_float((__float_as_uint(q2) & 0x7FFFFFFFu) | (__float_as_uint(x[i]) & 0x80000000u));
  }
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], lo, true);
}

// The same, exact path: IEEE division and the software conversion.
__device__ __forceinline__ uint32_t exact_pack4(float x0, float x1, float x2, float x3, float s) {
  return f32_to_e4m3_satfinite(x0 / s) | (f32_to_e4m3_satfinite(x1 / s) << 8) |
         (f32_to_e4m3_satfinite(x2 / s) << 16) | (f32_to_e4m3_satfinite(x3 / s) << 24);
}

// One pass of a wave: 16 elements per lane (a, b), 8 lanes per scale block;
// the e4m3 codes and this lane's block scale (wave-uniform fast/exact branch).
__device__ __forceinline__ void quantize_pass(const uint4& a, const uint4& b, uint4& out, float& s) {
  const uint32_t m = group8_max_u32(lane_absmax_bits(a, b));
  const bool odd = m > 0x7F7Fu || (m != 0u && m < kQTinyBf16);
  const uint32_t e[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  if (__ballot(odd) == 0) {
    const float amax = __uint_as_float(m << 16);
    s = amax > 0.0f ? amax / 448.0f : 1.0f;
    const float r = 1.0f / s;
    out.x = fast_pack4(bf16_lo(e[0]), bf16_hi(e[0]), bf16_lo(e[1]), bf16_hi(e[1]), s, r);
    out.y = fast_pack4(bf16_lo(e[2]), bf16_hi(e[2]), bf16_lo(e[3]), bf16_hi(e[3]), s, r);
    out.z = fast_pack4(bf16_lo(e[4]), bf16_hi(e[4]), bf16_lo(e[5]), bf16_hi(e[5]), s, r);
    out.w = fast_pack4(bf16_lo(e[6]), bf16_hi(e[6]), bf16_lo(e[7]), bf16_hi(e[7]), s, r);
  } else {
    const float amax = __uint_as_float(group8_max_u32(lane_absmax_bits_nonnan(a, b)) << 16);
    s = amax > 0.0f ? amax / 448.0f : 1.0f;
    out.x = exact_pack4(bf16_lo(e[0]), bf16_hi(e[0]), bf16_lo(e[1]), bf16_hi(e[1]), s);
    out.y = exact_pack4(bf16_lo(e[2]), bf16_hi(e[2]), bf16_lo(e[3]), bf16_hi(e[3]), s);
    out.z = exact_pack4(bf16_lo(e[4]), bf16_hi(e[4]), bf16_lo(e[5]), bf16_hi(e[5]), s);
    out.w = exact_pack4(bf16_lo(e[6]), bf16_hi(e[6]), bf16_lo(e[7]), bf16_hi(e[7]), s);
  }
}

__global__ void __launch_bounds__(kQThreads)
quantize_hidden_kernel(const uint16_t* __restrict__ x, int T, uint8_t* __restrict__ q,
                       float* __restrict__ scale) {
  __shared__ float sc[kNHBlk][kQTokens];
  const int w = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int t = blockIdx.x * kQTokens + w;
  if (t < T) {
    const uint16_t* row = x + (size_t)t * kH + lane * kQLaneCols;
    uint8_t* qrow = q + (size_t)t * kH + lane * kQLaneCols;
    // the whole row (14 x 16 B per lane) is in flight before any arithmetic
    uint4 raw[2 * kQPasses];
#pragma unroll
    for (int c = 0; c < kQPasses; ++c) {
      raw[2 * c] = *(const uint4*)(row + c * kQPass);
      raw[2 * c + 1] = *(const uint4*)(row + c * kQPass + 8);
    }
#pragma unroll
    for (int c = 0; c < kQPasses; ++c) {
      uint4 out;
      float s;
      quantize_pass(raw[2 * c], raw[2 * c + 1], out, s);
      *(uint4*)(qrow + c * kQPass) = out;
      if ((lane & (kQLanesPerBlk - 1)) == 0) sc[c * (kQPass / kBlk) + lane / kQLanesPerBlk][w] = s;
    }
  }
  __syncthreads();
  // scale[b][t0 .. t0+kQTokens-1]: contiguous floats per block row
  const int t0 = blockIdx.x * kQTokens;
  for (int i = threadIdx.x; i < kNHBlk * kQTokens; i += kQThreads) {
    const int b = i / kQTokens, k = i % kQTokens;
    if (t0 + k < T) scale[(size_t)b * T + t0 + k] = sc[b][k];
  }
}

// Small T (latency-bound with one wave per row): one workgroup per token
// row, wave p quantises pass p (columns 1024p ..) and writes its 8 block
// scales directly.  Same arithmetic as above, so the same bits.
constexpr int kQSmallMaxTokens = 2048;

__global__ void __launch_bounds__(kQPasses * kWave)
quantize_hidden_rows_kernel(const uint16_t* __restrict__ x, int T, uint8_t* __restrict__ q,
                            float* __restrict__ scale) {
  const int t = blockIdx.x;
  const int c = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const uint16_t* src = x + (size_t)t * kH + c * kQPass + lane * kQLaneCols;
  const uint4 a = *(const uint4*)src, b = *(const uint4*)(src + 8);
  uint4 out;
  float s;
  quantize_pass(a, b, out, s);
  *(uint4*)(q + (size_t)t * kH + c * kQPass + lane * kQLaneCols) = out;
  if ((lane & (kQLanesPerBlk - 1)) == 0) scale[(size_t)(c * (kQPass / kBlk) + lane / kQLanesPerBlk) * T + t] = s;
}

}  // namespace

hipError_t launch_quantize_hidden(const uint16_t* x, int T, uint8_t* q, float* scale, hipStream_t stream) {
  if (T <= kQSmallMaxTokens) {
    hipLaunchKernelGGL(quantize_hidden_rows_kernel, dim3(T), dim3(kQPasses * kWave), 0, stream, x, T, q, scale);
    return hipGetLastError();
  }
  const int blocks = (T + kQTokens - 1) / kQTokens;
  hipLaunchKernelGGL(quantize_hidden_kernel, dim3(blocks), dim3(kQThreads), 0, stream, x, T, q, scale);
  return hipGetLastError();
}

}  // namespace moe
