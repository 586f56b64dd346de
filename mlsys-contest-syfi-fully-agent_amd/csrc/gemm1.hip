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
// Token count from which GEMM1 uses the LDS-tiled MFMA kernel.
constexpr int kGemm1TiledMinTokens = 2048;
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

// ---------------------------------------------------------------------------
// Tiled path (many rows per expert): LDS-staged, MFMA-bound.
//
//   * workgroup = WM x WN waves; wave tile = (16*MI) rows x 64 MFMA columns,
//     i.e. 32 gate columns j..j+31 and the 32 matching up columns 2048+j..;
//     in the MFMA output layout a lane holds gate and up of the same (row,
//     column), so SwiGLU needs no data movement;
//   * one pipeline stage = one 128-wide K block (one scale block) of the A
//     rows (gathered tokens), the B rows (W13), and the A scales;
//   * stages are copied global -> LDS with global_load_lds_dwordx4 (no VGPR
//     staging), 3 LDS buffers, loads for stage kb+2 in flight while stage kb
//     is multiplied;
//   * LDS holds each 16-row x 128-K operand fragment as two 1 KB planes in the
//     MFMA register order (lane L = 16*q + r owns row r, K bytes 32q..32q+31),
//     so every ds_read_b128 of the MFMA operands is contiguous across the wave
//     (no bank conflicts) and every DMA writes one contiguous plane;
//   * per K block: P = A_f8 * B_f8 (v_mfma_f32_16x16x128_f8f6f4, exact
//     products), acc += P * (a_scale[row] * w_scale[n/128]).
// ---------------------------------------------------------------------------
template <int WM, int WN, int MI>
struct G1Tiled {
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = kWave * kWaves;
  static constexpr int BM = 16 * MI * WM;       // rows per tile
  static constexpr int kGateCols = 32 * WN;     // act columns per tile
  static constexpr int kNT = kI / kGateCols;    // column tiles
  static constexpr int kAFrags = BM / 16;
  static constexpr int kBFrags = 4 * WN;        // 2*WN gate + 2*WN up fragments
  static constexpr int kFrag = 2048;            // bytes of a 16 x 128 fp8 fragment
  static constexpr int kBOff = kAFrags * kFrag;
  static constexpr int kSOff = kBOff + kBFrags * kFrag;
  static constexpr int kStageBytes = kSOff + BM * 4;
  static constexpr int kStages = 3;
  static constexpr int kPlanes = 2 * (kAFrags + kBFrags);
  static_assert(kPlanes % kWaves == 0, "planes must split evenly over waves");
  static constexpr int kPlanesPerWave = kPlanes / kWaves;
  static constexpr int kScaleRowsPerWave = BM / kWaves;
  static_assert(kScaleRowsPerWave >= 1 && kScaleRowsPerWave <= kWave, "scale rows per wave");
  static constexpr int kDmaPerStage = kPlanesPerWave + 1;
  static constexpr int kGroupM = 4;             // row tiles per L2 group
};

template <int WM, int WN, int MI>
__global__ void __launch_bounds__(64 * WM * WN)
gemm1_tiled_kernel(const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale, int T,
                   const uint8_t* __restrict__ w13, const float* __restrict__ w13_scale,
                   const int32_t* __restrict__ expert_off, const int32_t* __restrict__ perm_token,
                   uint16_t* __restrict__ act) {
  using C = G1Tiled<WM, WN, MI>;
  __shared__ __attribute__((aligned(1024))) char lds[C::kStages * C::kStageBytes];

  // ---- tile of this workgroup ------------------------------------------
  const int mt_total = count_row_tiles(expert_off, C::BM);
  const int t = xcd_tile(blockIdx.x, mt_total * C::kNT);
  if (t < 0) return;
  int mt, nt;
  grouped_tile(t, mt_total, C::kNT, C::kGroupM, mt, nt);
  int e, row0, rows;
  find_row_tile(expert_off, mt, C::BM, e, row0, rows);
  const int j0 = nt * C::kGateCols;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform (SGPR)
  const int lane = threadIdx.x & (kWave - 1);
  const int lq = lane >> 4;
  const int lr = lane & 15;
  const int wm = wave / WN;
  const int wn = wave % WN;

  // ---- per-lane DMA sources (kb = 0) -------------------------------------
  const uint8_t* src[C::kPlanesPerWave];
  int dst[C::kPlanesPerWave];
#pragma unroll
  for (int k = 0; k < C::kPlanesPerWave; ++k) {
    const int plane = wave + k * C::kWaves;
    const int frag = plane >> 1, half = plane & 1;
    const int kofs = 32 * lq + 16 * half;
    if (frag < C::kAFrags) {
      const int r = min(frag * 16 + lr, rows - 1);
      src[k] = hs + (size_t)perm_token[row0 + r] * kH + kofs;
      dst[k] = frag * C::kFrag + half * 1024;
    } else {
      const int bf = frag - C::kAFrags;
      const int n = bf < 2 * WN ? j0 + 16 * bf + lr : kI + j0 + 16 * (bf - 2 * WN) + lr;
      src[k] = w13 + ((size_t)e * k2I + n) * kH + kofs;
      dst[k] = C::kBOff + bf * C::kFrag + half * 1024;
    }
  }
  const int srow = wave * C::kScaleRowsPerWave + lane;
  const float* ssrc = hs_scale + perm_token[row0 + min(srow, rows - 1)];
  const bool sload = lane < C::kScaleRowsPerWave;
  const int sdst = C::kSOff + wave * C::kScaleRowsPerWave * 4;

  auto issue = [&](int kb) {
    char* base = lds + (kb % C::kStages) * C::kStageBytes;
#pragma unroll
    for (int k = 0; k < C::kPlanesPerWave; ++k) dma16(src[k] + kb * kBlk, base + dst[k]);
    if (sload) dma4(ssrc + (size_t)kb * T, base + sdst);
  };

  // weight block scales of this wave's gate / up columns
  const float* sg_ptr = w13_scale + ((size_t)e * kN2IBlk + (j0 + 32 * wn) / kBlk) * kNHBlk;
  const float* su_ptr = w13_scale + ((size_t)e * kN2IBlk + (kI + j0 + 32 * wn) / kBlk) * kNHBlk;

  v4f acc[MI][4];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) acc[mi][nj] = v4f{0.f, 0.f, 0.f, 0.f};

  issue(0);
  issue(1);
#pragma unroll 1
  for (int kb = 0; kb < kNHBlk; ++kb) {
    if (kb + 1 < kNHBlk)
      wait_vmcnt_lgkm0<C::kDmaPerStage>();
    else
      wait_vmcnt_lgkm0<0>();
    block_barrier();
    if (kb + 2 < kNHBlk) issue(kb + 2);

    const char* sb = lds + (kb % C::kStages) * C::kStageBytes;
    v8i a[MI], b[4];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      const char* f = sb + (wm * MI + mi) * C::kFrag + lane * 16;
      const v4i lo = *(const v4i*)f, hi = *(const v4i*)(f + 1024);
      a[mi] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) {
      const int bf = nj < 2 ? 2 * wn + nj : 2 * WN + 2 * wn + (nj - 2);
      const char* f = sb + C::kBOff + bf * C::kFrag + lane * 16;
      const v4i lo = *(const v4i*)f, hi = *(const v4i*)(f + 1024);
      b[nj] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
    const float sg = sg_ptr[kb], su = su_ptr[kb];
    v4f sgm[MI], sum[MI];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      const v4f sa = *(const v4f*)(sb + C::kSOff + (wm * 16 * MI + 16 * mi + 4 * lq) * 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sgm[mi][i] = sa[i] * sg;
        sum[mi][i] = sa[i] * su;
      }
    }
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int nj = 0; nj < 4; ++nj) {
        const v4f p = mfma_f8_16x16x128(a[mi], b[nj]);
        const v4f s = nj < 2 ? sgm[mi] : sum[mi];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mi][nj][i] = __builtin_fmaf(p[i], s[i], acc[mi][nj][i]);
      }
  }

  // ---- SwiGLU epilogue (moe.py:190-193): act = silu(up) * gate ------------
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int nj = 0; nj < 2; ++nj)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = (wm * MI + mi) * 16 + 4 * lq + i;
        if (r < rows) {
          const float x1 = acc[mi][nj][i], x2 = acc[mi][nj + 2][i];
          const float silu = x2 / (1.0f + expf(-x2));
          act[(size_t)(row0 + r) * kI + j0 + 32 * wn + 16 * nj + lr] = f32_to_bf16_rne(silu * x1);
        }
      }
}

template <int WM, int WN, int MI>
hipError_t launch_gemm1_tiled(const uint8_t* hs, const float* hs_scale, int T, const uint8_t* w13,
                              const float* w13_scale, const Layout& L, char* ws, hipStream_t stream) {
  using C = G1Tiled<WM, WN, MI>;
  const int64_t pairs = (int64_t)T * kTopK;
  const int64_t mtiles = (pairs + C::BM - 1) / C::BM + (pairs < kELocal ? pairs : kELocal);
  const int64_t blocks = ((mtiles * C::kNT + 7) / 8) * 8;
  hipLaunchKernelGGL((gemm1_tiled_kernel<WM, WN, MI>), dim3((unsigned)blocks), dim3(C::kThreads), 0,
                     stream, hs, hs_scale, T, w13, w13_scale, (const int32_t*)(ws + L.expert_off),
                     (const int32_t*)(ws + L.perm_token), (uint16_t*)(ws + L.act));
  return hipGetLastError();
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
  if (T < kGemm1TiledMinTokens)
    return launch_gemm1_cfg<4, 4>(hs, hs_scale, T, w13, w13_scale, L, ws, max_row_tiles(T, 64), stream);
  return launch_gemm1_tiled<4, 2, 4>(hs, hs_scale, T, w13, w13_scale, L, ws, stream);
}

}  // namespace moe
