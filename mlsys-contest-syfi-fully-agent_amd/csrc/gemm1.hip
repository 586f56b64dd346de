// gemm1.hip -- grouped FP8 GEMM1 (hidden 7168 -> gate/up 4096) with the
// per-128-K block-scale dequantisation folded into the fp32 accumulator and
// SwiGLU fused into the epilogue; writes the bf16 activation rows GEMM2 reads.
//
// Reference behaviour: moe.py:186-193 (G1 = A_e W13_e^T; C = silu(G1[:, I:]) *
// G1[:, :I]); CUDA solution gemm_fp8_fp8_grouped_kernel (moe.cu:1373-1609) and
// swiglu_kernel (moe.cu:2125-2146), which round-trip G1 through fp32 HBM.
//
// Design (gfx950):
//   * v_mfma_f32_16x16x128_f8f6f4 covers exactly one 128-wide K scale block per
//     instruction, so each MFMA yields the unscaled block partial P and the
//     accumulator takes  acc += P * (a_scale[row, kb] * w_scale[n/128, kb]).
//     fp8 x fp8 products are exact; only fp32 summation order differs from the
//     fp32 reference.
//   * each 16-column MFMA tile packs 8 gate columns (n0..n0+7) and the 8
//     matching up columns (2048+n0..): the SwiGLU epilogue is one xor-8 lane
//     shuffle, and a tile only needs 8 output columns, so even a single-token
//     expert spreads over 256 workgroups (the HBM-bound decode case).
//   * operands go straight from global memory into the MFMA register layout
//     (both A and W13 are K-contiguous, so no transpose and no LDS staging);
//     the token gather is fused into the A load (row -> perm_token -> hidden).
//   * the 4 waves of a workgroup split the 56 K blocks; partials are summed
//     through LDS before the epilogue.
#include "moe_common.hpp"

namespace moe {
namespace {

constexpr int kG1Threads = 256;
constexpr int kG1Waves = kG1Threads / kWave;

template <int MI, int NJ>
__global__ void __launch_bounds__(kG1Threads)
gemm1_swiglu_kernel(const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale, int T,
                    const uint8_t* __restrict__ w13, const float* __restrict__ w13_scale,
                    const int32_t* __restrict__ expert_off, const int32_t* __restrict__ perm_token,
                    uint16_t* __restrict__ act) {
  constexpr int BM = 16 * MI;
  int e, row0, rows;
  if (!find_row_tile(expert_off, blockIdx.y, BM, e, row0, rows)) return;

  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int lr = lane & 15;  // operand row / output column inside a 16x16 tile
  const int lq = lane >> 4;  // K quarter (operands) / output row group

  // A operand rows (gathered tokens); rows past the tile end repeat the last
  // valid row so every load stays in bounds (their outputs are discarded).
  const uint8_t* a_ptr[MI];
  int out_tok[MI][4];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
    const int tok = perm_token[row0 + min(mi * 16 + lr, rows - 1)];
    a_ptr[mi] = hs + (size_t)tok * kH + lq * 32;
#pragma unroll
    for (int i = 0; i < 4; ++i) out_tok[mi][i] = perm_token[row0 + min(mi * 16 + lq * 4 + i, rows - 1)];
  }
  // B operand rows: packed gate/up columns.
  const uint8_t* b_ptr[NJ];
  const float* bs_ptr[NJ];
#pragma unroll
  for (int nj = 0; nj < NJ; ++nj) {
    const int n0 = (blockIdx.x * NJ + nj) * 8;
    const int n = lr < 8 ? n0 + lr : kI + n0 + (lr - 8);
    b_ptr[nj] = w13 + ((size_t)e * k2I + n) * kH + lq * 32;
    bs_ptr[nj] = w13_scale + ((size_t)e * kN2IBlk + n / kBlk) * kNHBlk;
  }

  v4f acc[MI][NJ];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) acc[mi][nj] = v4f{0.f, 0.f, 0.f, 0.f};

#pragma unroll 2
  for (int kb = wave; kb < kNHBlk; kb += kG1Waves) {
    v8i a[MI], b[NJ];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) a[mi] = *(const v8i*)(a_ptr[mi] + kb * kBlk);
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) b[nj] = *(const v8i*)(b_ptr[nj] + kb * kBlk);
    float sa[MI][4], sw[NJ];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int i = 0; i < 4; ++i) sa[mi][i] = hs_scale[(size_t)kb * T + out_tok[mi][i]];
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) sw[nj] = bs_ptr[nj][kb];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj) {
        const v4f p = mfma_f8_16x16x128(a[mi], b[nj]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mi][nj][i] = __builtin_fmaf(p[i], sa[mi][i] * sw[nj], acc[mi][nj][i]);
      }
  }

  // Sum the K-split partials of the 4 waves.
  __shared__ float red[kG1Waves - 1][MI * NJ * 4][kWave];
  if (wave > 0) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave - 1][(mi * NJ + nj) * 4 + i][lane] = acc[mi][nj][i];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < kG1Waves - 1; ++w)
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mi][nj][i] += red[w][(mi * NJ + nj) * 4 + i][lane];

  // SwiGLU (moe.py:190-193): lanes lr < 8 hold gate columns, lanes lr + 8 the
  // matching up columns.
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) {
      const int n0 = (blockIdx.x * NJ + nj) * 8;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x1 = acc[mi][nj][i];
        const float x2 = __shfl_xor(x1, 8, kWave);
        const int r = mi * 16 + lq * 4 + i;
        if (lr < 8 && r < rows) {
          const float silu = x2 / (1.0f + expf(-x2));
          act[(size_t)(row0 + r) * kI + n0 + lr] = f32_to_bf16_rne(silu * x1);
        }
      }
    }
}

template <int MI, int NJ>
hipError_t launch_gemm1_cfg(const uint8_t* hs, const float* hs_scale, int T, const uint8_t* w13,
                            const float* w13_scale, const Layout& L, char* ws, int max_tiles,
                            hipStream_t stream) {
  const dim3 grid(kI / (8 * NJ), max_tiles);
  hipLaunchKernelGGL((gemm1_swiglu_kernel<MI, NJ>), grid, dim3(kG1Threads), 0, stream, hs, hs_scale,
                     T, w13, w13_scale, (const int32_t*)(ws + L.expert_off),
                     (const int32_t*)(ws + L.perm_token), (uint16_t*)(ws + L.act));
  return hipGetLastError();
}

// Upper bound on the number of row tiles of height bm over all experts.
inline int max_row_tiles(int T, int bm) {
  const int64_t pairs = (int64_t)T * kTopK;
  const int64_t bound = (pairs + bm - 1) / bm + (pairs < kELocal ? pairs : kELocal);
  return (int)(bound < pairs ? bound : pairs);
}

}  // namespace

hipError_t launch_gemm1(const uint8_t* hs, const float* hs_scale, int T, const uint8_t* w13,
                        const float* w13_scale, const Layout& L, char* ws, hipStream_t stream) {
  if (T <= 8) return launch_gemm1_cfg<1, 1>(hs, hs_scale, T, w13, w13_scale, L, ws, max_row_tiles(T, 16), stream);
  return launch_gemm1_cfg<4, 4>(hs, hs_scale, T, w13, w13_scale, L, ws, max_row_tiles(T, 64), stream);
}

}  // namespace moe
