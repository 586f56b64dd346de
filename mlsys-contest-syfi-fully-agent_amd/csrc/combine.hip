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

// A workgroup of kCombThreads threads (one wave) combines 256 * kChunks
// columns of one token: thread i takes columns 256 h + 4i .. +3 of its part
// for h < kChunks, so each load instruction of a wave covers 1 KB of
// contiguous bytes.  The token's rows are added in batches of kBatch rows,
// every lane issuing a batch's (kBatch x kChunks) 16-byte loads of fp32 GEMM2
// rows before its first add.  The rows are read once, with nontemporal loads
// (at T = 8192: 201 -> 183 us).  Many small workgroups per CU overlap their
// index loads with other tokens' row loads (interleaved runs, T = 4096 / 8192
// / 14107: 93.2 / 183.3 / 318.7 us with one 896-thread workgroup per token,
// 89.9 / 179.0 / 311.5 with 64 threads; 448 and 128 threads in between).
// Two shapes, same bits:
//   * kChunks = 2, kBatch = 8 (14 workgroups per token): every row of the
//     token in one batch;
//   * kChunks = 4, kBatch = 4 (7 per token), from T = 2048 on, where experts
//     of every token leave most tokens one or two rows: twice the loads in
//     flight per lane for such tokens.  Interleaved A/B, combine us, hot
//     experts: T = 8192 72.9 -> 67.3, 4096 40.0 -> 37.2, 2048 22.8 -> 22.5;
//     prefill routing T = 8192 64.3 -> 64.1; at T = 1024 it lost 0.4-0.9 us.
constexpr int kCombThreads = 64;
constexpr int kCombWideMinTokens = 2048;

template <int kChunks, int kBatch>
__global__ void __launch_bounds__(kCombThreads)
combine_kernel(const float* __restrict__ down, const int32_t* __restrict__ pair_row,
               const float* __restrict__ topk_w, const int32_t* __restrict__ expert_off, int T,
               uint16_t* __restrict__ out) {
  constexpr int kCombCols = 4 * kChunks * kCombThreads;
  constexpr int kCombParts = kH / kCombCols;
  static_assert(kCombParts * kCombCols == kH && kCombThreads == kWave, "one wave, whole parts");
  const int t = blockIdx.x / kCombParts;
  const int c0 = (blockIdx.x % kCombParts) * kCombCols + (int)threadIdx.x * 4;
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
  // The token's rows to add, in pick (ascending expert) order, batch by batch.
  uint32_t m = 0;
#pragma unroll
  for (int k = 0; k < kTopK; ++k) m |= (row[k] >= 0 ? 1u : 0u) << k;
  const int n = __builtin_popcount(m);
  float a[kChunks][4] = {};
#pragma unroll 1
  for (int b0 = 0; b0 < n; b0 += kBatch) {
    int rr[kBatch];
    float ww[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      if constexpr (kBatch >= kTopK) {  // one batch: the picks in place
        rr[j] = row[j];
        ww[j] = w[j];
        continue;
      }
      // pick k of the (b0 + j)-th row, selected without indexing the registers
      const int k = b0 + j < n ? nth_set_bit(m, b0 + j) : 0;
      int r = row[0];
      float x = w[0];
#pragma unroll
      for (int kk = 1; kk < kTopK; ++kk) {
        r = k == kk ? row[kk] : r;
        x = k == kk ? w[kk] : x;
      }
      rr[j] = b0 + j < n ? r : -1;
      ww[j] = x;
    }
    v4f v[kBatch][kChunks];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      if (rr[j] < 0) continue;  // token-uniform
      const float* src = down + (size_t)rr[j] * kH + c0;
#pragma unroll
      for (int h = 0; h < kChunks; ++h) v[j][h] = __builtin_nontemporal_load((const v4f*)(src + h * 256));
    }
    // ascending expert order, acc = acc + (O * w): two roundings, as index_add_
    // of O * w in moe.py:199-200
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      if (rr[j] < 0) continue;
#pragma unroll
      for (int h = 0; h < kChunks; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) a[h][i] = a[h][i] + v[j][h][i] * ww[j];
    }
  }
#pragma unroll
  for (int h = 0; h < kChunks; ++h) {
    const uint2 o{(uint32_t)f32_to_bf16_rne(a[h][0]) | ((uint32_t)f32_to_bf16_rne(a[h][1]) << 16),
                  (uint32_t)f32_to_bf16_rne(a[h][2]) | ((uint32_t)f32_to_bf16_rne(a[h][3]) << 16)};
    *(uint2*)(out + (size_t)t * kH + c0 + h * 256) = o;
  }
}

template <int kChunks, int kBatch>
hipError_t launch_combine_shape(int T, const Layout& L, char* ws, void* out, hipStream_t stream) {
  hipLaunchKernelGGL((combine_kernel<kChunks, kBatch>), dim3(T * (kH / (256 * kChunks))), dim3(kCombThreads), 0,
                     stream, (const float*)(ws + L.down), (const int32_t*)(ws + L.pair_row),
                     (const float*)(ws + L.topk_w), (const int32_t*)(ws + L.expert_off), T, (uint16_t*)out);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_combine(int T, const Layout& L, char* ws, void* out, hipStream_t stream) {
  return T >= kCombWideMinTokens ? launch_combine_shape<4, 4>(T, L, ws, out, stream)
                                 : launch_combine_shape<2, 8>(T, L, ws, out, stream);
}

}  // namespace moe
