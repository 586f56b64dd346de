// gemm2.hip -- grouped GEMM2 (activation 2048 -> hidden 7168) with the
// per-128x128 weight block scale folded into the fp32 accumulator.
//
// Reference behaviour: moe.py:195-196 (O = C W2_e^T with C in fp32); CUDA
// solution gemm_fp32_fp8w_fused_acc_grouped_kernel (moe.cu:2186-2431), which
// emulates fp32 A with hi/lo bf16 pairs.
//
// Precision: the activation C arrives as a bf16 (hi, lo) pair (hi + lo
// carries the fp32 SwiGLU value to ~2^-17) and the e4m3 weights are widened
// exactly to bf16, so every product of the fp32 reference is formed: two
// v_mfma_f32_16x16x32_bf16 per operand pair, fp32 accumulation (this MFMA
// sums to fp32 accuracy; the fp8 one does not -- see gemm1.hip).  That is the
// reference CUDA's own hi/lo design; a single bf16 C fails the 1e-2 check on
// several percent of the elements once outputs reach ~1e3.
//
// Two kernels: a streaming one for T <= 64 (weights read once, the
// routing-weighted combine fused in) and an LDS-tiled one for larger T (fp32
// rows to the combine pass).
#include <type_traits>

#include "kernels.hpp"

namespace moe {
namespace {

// ---------------------------------------------------------------------------
// Streaming path with the combine fused in (T <= kGemm2StreamMaxTokens).
//
//   * a workgroup owns 32 output columns n0..n0+31 for all T tokens; it walks
//     the active experts in ascending order (the order of moe.py:168-200) and
//     their 16-row tiles, computing O = act_rows . W2_e[n0..n0+31]^T
//     (two 16-column MFMA blocks: each job's act rows are loaded once for
//     32 columns, which halves their L2 traffic against 16-column groups);
//   * its 8 waves split K (2 scale blocks each); the W2 slices of the next
//     two (expert, row tile) jobs stream into LDS while one is multiplied;
//   * the K-partials are summed in LDS in a fixed order and each row's
//     O * weight is added to its token's fp32 accumulator in LDS
//     (acc = acc + O * w, the two roundings of moe.py:199-200); a token occurs
//     at most once per expert, so no atomics are needed and the result is
//     deterministic;
//   * finally every token's 32 columns are rounded to bf16 and stored (tokens
//     without a local expert get zeros).  No GEMM2 rows reach HBM and no
//     separate combine pass runs.
// ---------------------------------------------------------------------------
constexpr int kS2Waves = 8;
constexpr int kS2Threads = kS2Waves * kWave;
constexpr int kS2KB = kNIBlk / kS2Waves;  // 2 scale blocks per wave
constexpr int kS2NB = 2;                  // 16-column blocks per workgroup
constexpr int kS2Cols = 16 * kS2NB;       // output columns per workgroup
constexpr int kS2Units = kH / kS2Cols;    // 224 column groups
static_assert(kBlk % kS2Cols == 0, "a workgroup's columns share one weight scale block");

struct S2Job {
  int e, rt;  // expert, row tile; e < 0: none
};

// Next (expert, row tile) after `j` in ascending expert order (wave-level).
__device__ __forceinline__ S2Job s2_next(const ExpertRows& X, uint32_t active, S2Job j) {
  if (j.e >= 0 && (j.rt + 1) * 16 < X.end(j.e) - X.begin(j.e)) return {j.e, j.rt + 1};
  const uint32_t later = j.e >= 0 ? active & ~((2u << j.e) - 1u) : active;
  return later ? S2Job{__builtin_ctz(later), 0} : S2Job{-1, 0};
}

// A job's act operands, 16 slots: slot c = ((k * 2 + g) * 2 + h) * 2 + part
// holds, in lane (q, r), row r's columns (kb0 + k) * 128 + 64 g + 16 q + 8 h
// .. +7 (64-column chunk 2 (kb0 + k) + g), the bf16 hi half (part 0) or the
// lo half (part 1, 64 elements further in the act row).
static_assert(kS2KB == 2, "16 act operand slots per job");
constexpr int kS2Slots = 8 * kS2KB;
constexpr int s2_slot(int k, int g, int h, int part) { return ((k * 2 + g) * 2 + h) * 2 + part; }
__device__ __forceinline__ int s2_slot_off(int c) {
  return (2 * (c >> 3) + ((c >> 2) & 1)) * 128 + 8 * ((c >> 1) & 1) + 64 * (c & 1);
}

struct S2Regs {
  v4i op[kS2Slots];  // act operands (spread S > 0: over op[0 .. 16 / 2^S), see s2_load)
  float sw[kS2KB];
  int tok;           // token and weight of the row this thread combines
  float pw;          //   (row = (tid / 16) % 16 of the tile)
};

// Loads a job's act rows.  The loads cost per instruction, not per lane: a
// job of one to four rows took 16 of them for 16 rows, on the path its W2
// copies share (small_t64: 18 of GEMM2's 63 us).  Spread S: every expert of
// the launch has at most 16 / 2^S rows (so every job), and the 16 slots take
// 16 / 2^S instructions, lane (q, r) taking row r mod 16 / 2^S of slot
// 2^S i + r / (16 / 2^S) (S = 2: row r % 4 of slot 4i + r / 4); s2_operand
// moves them into the MFMA lanes once they have landed.  Chosen per launch,
// not per job: a branch per job made the compiler merge two layouts of the
// persistent operand registers and wait for every load in flight before the
// next job's loads.
template <int S>
__device__ __forceinline__ void s2_load(S2Regs& R, S2Job j, const ExpertRows& X,
                                        const int32_t* __restrict__ perm_token, const float* __restrict__ perm_w,
                                        const uint16_t* __restrict__ act, const float* __restrict__ w2_scale, int n0,
                                        int kb0, int lq, int lr) {
  const int row0 = X.begin(j.e) + j.rt * 16;
  const int rows = min(16, X.end(j.e) - row0);
  // combine operands first: waiting for them never waits for the prefetch
  const int crow = row0 + min((int)(threadIdx.x >> 4) & 15, rows - 1);
  R.tok = perm_token[crow];
  R.pw = perm_w[crow];
  const uint16_t* ab = act + (size_t)kb0 * 256 + 16 * lq;  // + row * kActRowElems + s2_slot_off(slot)
  constexpr int kRows = 16 >> S;  // rows one load instruction covers
  const uint16_t* ap = ab + (size_t)(row0 + min(lr & (kRows - 1), rows - 1)) * kActRowElems;
#pragma unroll
  for (int i = 0; i < kS2Slots >> S; ++i) R.op[i] = *(const v4i*)(ap + s2_slot_off((i << S) + lr / kRows));
#pragma unroll
  for (int k = 0; k < kS2KB; ++k) R.sw[k] = w2_scale[((size_t)j.e * kNHBlk + n0 / kBlk) * kNIBlk + kb0 + k];
}

// v4i of lane r + N of the lane's 16-lane row (DPP row_shl:N; lanes past the
// row's end read 0 and feed only discarded rows).
template <int N>
__device__ __forceinline__ v4i row_shl(const v4i& x) {
  if constexpr (N == 0) {
    return x;
  } else {
    return v4i{__builtin_amdgcn_mov_dpp(x[0], 0x100 + N, 0xF, 0xF, true),
               __builtin_amdgcn_mov_dpp(x[1], 0x100 + N, 0xF, 0xF, true),
               __builtin_amdgcn_mov_dpp(x[2], 0x100 + N, 0xF, 0xF, true),
               __builtin_amdgcn_mov_dpp(x[3], 0x100 + N, 0xF, 0xF, true)};
  }
}

// Operand slot C of a landed job in the MFMA layout (lane (q, r): row r);
// spread S: slot C sits in op[C / 2^S], lanes shifted by (C mod 2^S) * 16 /
// 2^S.  Template constants: a shift chosen at run time (folded only after
// unrolling) left the operands in scratch memory.
template <int S, int C>
__device__ __forceinline__ v4i s2_operand(const S2Regs& R) {
  return row_shl<(C & ((1 << S) - 1)) * (16 >> S)>(R.op[C >> S]);
}

// s2_operand for the unrolled (k, g, h, part) of the MFMA loop: the 16 slot
// constants spelled out, so that every shift is a template constant.
template <int S>
__device__ __forceinline__ v4i s2_op(const S2Regs& R, int k, int g, int h, int part) {
  switch (s2_slot(k, g, h, part)) {
    case 0: return s2_operand<S, 0>(R);
    case 1: return s2_operand<S, 1>(R);
    case 2: return s2_operand<S, 2>(R);
    case 3: return s2_operand<S, 3>(R);
    case 4: return s2_operand<S, 4>(R);
    case 5: return s2_operand<S, 5>(R);
    case 6: return s2_operand<S, 6>(R);
    case 7: return s2_operand<S, 7>(R);
    case 8: return s2_operand<S, 8>(R);
    case 9: return s2_operand<S, 9>(R);
    case 10: return s2_operand<S, 10>(R);
    case 11: return s2_operand<S, 11>(R);
    case 12: return s2_operand<S, 12>(R);
    case 13: return s2_operand<S, 13>(R);
    case 14: return s2_operand<S, 14>(R);
    default: return s2_operand<S, 15>(R);
  }
}


// A job's W2 bytes of this wave (rows n0 .. n0 + 31, K blocks kb0, kb0 + 1)
// -> the wave's LDS stage: per 16-row block and K block two wide planes (rows
// 0-7, 8-15), 128 bytes per row, chunks swizzled, so every copy reads 8 whole
// 128-byte row segments.  8 copies per lane.
__device__ __forceinline__ void s2_copy_w(char* stage, S2Job j, const ExpertRows& X, const uint8_t* __restrict__ w2,
                                          int n0, int kb0, int lane) {
  auto copy = [&](auto nt_c) {
#pragma unroll
    for (int nb = 0; nb < kS2NB; ++nb)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        int r, c;
        wide_copy_lane(lane, h, r, c);
        const uint8_t* src = w2 + ((size_t)j.e * kH + n0 + 16 * nb + r) * kI + kb0 * kBlk + 16 * c;
#pragma unroll
        for (int k = 0; k < kS2KB; ++k) {
          if constexpr (decltype(nt_c)::value)
            dma16_nt(src + k * kBlk, stage + ((nb * kS2KB + k) * 2 + h) * 1024);
          else
            dma16(src + k * kBlk, stage + ((nb * kS2KB + k) * 2 + h) * 1024);
        }
      }
  };
  // A row tile with more of the expert's row tiles after it: the next job
  // copies the same W2 slice again, so the lines stay in L2 for it; the
  // expert's last row tile reads them for the last time.
  if ((j.rt + 1) * 16 < X.end(j.e) - X.begin(j.e))
    copy(std::false_type{});
  else
    copy(std::true_type{});
}

__global__ void __launch_bounds__(kS2Threads)
gemm2_combine_kernel(const uint16_t* __restrict__ act, const uint8_t* __restrict__ w2,
                     const float* __restrict__ w2_scale, const int32_t* __restrict__ expert_off,
                     const int32_t* __restrict__ perm_token, const float* __restrict__ perm_w, int T,
                     uint16_t* __restrict__ out) {
  // One LDS object (a second __shared__ array makes the compiler wait for
  // every LDS DMA before any LDS read): per wave a two-stage W2 ring, then
  // the token accumulators and the K-partials.
  constexpr int kStage = kS2NB * kS2KB * 2 * 1024;         // 8 KB per wave and job
  constexpr int kRing = 2 * kS2Waves * kStage;
  constexpr int kAccOff = kRing;
  constexpr int kRedOff = kAccOff + kGemm2StreamMaxTokens * kS2Cols * 4;
  constexpr int kLdsBytes = kRedOff + kS2Waves * kS2NB * 256 * 4;
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes];
  float* outacc = (float*)(lds + kAccOff);  // [token][32]
  float* red = (float*)(lds + kRedOff);     // [wave][column block][256]
  const int n0 = blockIdx.x * kS2Cols;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x & (kWave - 1);
  const int lq = lane >> 4;
  const int lr = lane & 15;
  const int kb0 = wave * kS2KB;
  auto stage = [&](int s) { return lds + (s * kS2Waves + wave) * kStage; };
  for (int i = threadIdx.x; i < T * kS2Cols; i += kS2Threads) outacc[i] = 0.f;

  ExpertRows X;
  X.load(expert_off);
  const uint32_t active = X.active();
  // Jobs in ascending (expert, row tile) order.  The W2 slices of the next
  // two jobs stream into the wave's two LDS stages while one is multiplied;
  // the act rows of the next job load into registers.
  //
  // Act rows are loaded only together with a W2 copy after them (when no job
  // after next exists, a second copy of the job just copied, whose lines are
  // in flight or in L2), so the act rows of every job are older than the
  // last 8 loads when its step starts.  The compiler's own wait before the
  // MFMAs counts, along every path, the loads issued after the operands';
  // with a copy that could be skipped alone it merged the paths to vmcnt(0)
  // and so waited for the prefetch it had just issued, one full memory
  // latency per job (small_t64: 3.6 us per job, 2.1 of it that wait).
  // Every expert of the launch has at most four rows (every launch at T <= 4,
  // decode among them) or at most eight: act rows spread over 4 or 8 loads
  // per job (s2_load), one loop for the whole launch (decode_t1_s3 23.7 ->
  // 22.6 us, T = 17 84.8 -> 79.0 us, same bits).
  const int spread = __ballot(X.cnt > 4) == 0 ? 2 : __ballot(X.cnt > 8) == 0 ? 1 : 0;
  auto run = [&](auto spread_c) {
    constexpr int S = decltype(spread_c)::value;
    S2Job job = s2_next(X, active, {-1, 0});
    S2Job j1 = job.e >= 0 ? s2_next(X, active, job) : job;
    S2Regs r0, r1;
    if (job.e >= 0) {
      s2_load<S>(r0, job, X, perm_token, perm_w, act, w2_scale, n0, kb0, lq, lr);
      s2_copy_w(stage(0), job, X, w2, n0, kb0, lane);
      s2_copy_w(stage(1), j1.e >= 0 ? j1 : job, X, w2, n0, kb0, lane);
    }
    // One job from stage `s` with act rows `cur`; after its MFMAs, loads the
    // next job's act rows into `nxt` and starts the copy of the job after next
    // into stage `s`.  Issue order is always: act rows of job j, copy of job
    // j + 1.
    auto step = [&](int s, const S2Regs& cur, S2Regs& nxt) {
      // This job's W2 stage and act rows have landed; the next job's W2 copy
      // (8 per lane, issued last) may stay in flight.
      wait_vmcnt_lgkm0<2 * kS2KB * kS2NB>();
      asm volatile("" ::: "memory");
      v4i b[kS2NB][kS2KB][2];
  #pragma unroll
      for (int nb = 0; nb < kS2NB; ++nb)
  #pragma unroll
        for (int k = 0; k < kS2KB; ++k)
  #pragma unroll
          for (int g = 0; g < 2; ++g)
            b[nb][k][g] = *(const v4i*)(stage(s) + 2 * (nb * kS2KB + k) * 1024 + wide_slot(lr, 4 * g + lq));
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the stage is read: free for the job after next
      const S2Job j2 = j1.e >= 0 ? s2_next(X, active, j1) : j1;
  #pragma unroll
      for (int nb = 0; nb < kS2NB; ++nb) {
        v4f acc = {0.f, 0.f, 0.f, 0.f};
  #pragma unroll
        for (int k = 0; k < kS2KB; ++k) {
          v4f p = {0.f, 0.f, 0.f, 0.f};
  #pragma unroll
          for (int g = 0; g < 2; ++g) {
            const v8bf b0 = e4m3x8_to_bf16((uint32_t)b[nb][k][g][0], (uint32_t)b[nb][k][g][1]);
            const v8bf b1 = e4m3x8_to_bf16((uint32_t)b[nb][k][g][2], (uint32_t)b[nb][k][g][3]);
            p = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, s2_op<S>(cur, k, g, 0, 0)), b0, p);
            p = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, s2_op<S>(cur, k, g, 1, 0)), b1, p);
            p = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, s2_op<S>(cur, k, g, 0, 1)), b0, p);
            p = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, s2_op<S>(cur, k, g, 1, 1)), b1, p);
          }
  #pragma unroll
          for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(p[i], cur.sw[k], acc[i]);
        }
  #pragma unroll
        for (int i = 0; i < 4; ++i) red[(wave * kS2NB + nb) * 256 + (4 * lq + i) * 16 + lr] = acc[i];
      }
      // The next job's loads go out after this job's MFMAs: with the memory
      // queue full their issue stalls, and the MFMAs no longer wait behind it
      // (small_t64 GEMM2 62.5 -> 61.5 us).
      if (j1.e >= 0) {
        s2_load<S>(nxt, j1, X, perm_token, perm_w, act, w2_scale, n0, kb0, lq, lr);
        s2_copy_w(stage(s), j2.e >= 0 ? j2 : j1, X, w2, n0, kb0, lane);
      }
      lds_barrier();
      {
        // thread = (column block nb, row r, column c): every thread of the workgroup
        static_assert(kS2Threads == kS2NB * 256, "one thread per output of a job");
        const int nb = threadIdx.x >> 8, r = (threadIdx.x >> 4) & 15, c = threadIdx.x & 15;
        const int row = X.begin(job.e) + job.rt * 16 + r;
        if (row < X.end(job.e)) {
          float o = red[nb * 256 + (threadIdx.x & 255)];
  #pragma unroll
          for (int w = 1; w < kS2Waves; ++w) o += red[(w * kS2NB + nb) * 256 + (threadIdx.x & 255)];
          const float p = o * cur.pw;
          float& a = outacc[cur.tok * kS2Cols + 16 * nb + c];
          a = a + p;
        }
      }
      lds_barrier();
      job = j1;
      j1 = j2;
    };
  #pragma unroll 1
    while (job.e >= 0) {
      step(0, r0, r1);
      if (job.e < 0) break;
      step(1, r1, r0);
    }
  };
  if (spread == 2)
    run(std::integral_constant<int, 2>{});
  else if (spread == 1)
    run(std::integral_constant<int, 1>{});
  else
    run(std::integral_constant<int, 0>{});
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the repeated copy lands before the LDS is released
  for (int i = threadIdx.x; i < T * kS2Cols; i += kS2Threads)
    out[(size_t)(i / kS2Cols) * kH + n0 + (i % kS2Cols)] = f32_to_bf16_rne(outacc[i]);
}

// ---------------------------------------------------------------------------
// Tiled path (many rows per expert): LDS-staged bf16 MFMA.
//
//   * workgroup = WM x WN waves, wave tile (16*MI) rows x (16*NJ) columns;
//   * a pipeline stage is 64 K values: the bf16 activation rows (A) and the
//     e4m3 W2 rows (B), copied global -> LDS by global_load_lds_dwordx4,
//     a ring of STAGES LDS buffers (shipped: two, the copy of stage s+1 in
//     flight while stage s multiplies);
//   * operand fragments sit in LDS row-major with swizzled chunks: an A
//     fragment (16 rows x 64 K bf16 = 128 B per row) is two wide planes, a B
//     fragment (16 rows x 64 K e4m3) one narrow plane; MFMA lane L = 16*q + r
//     works on row r, K = 16q .. 16q+15 of the stage, instruction j taking
//     K = 16q + 8j .. +7;
//   * B is widened e4m3 -> bf16 exactly in registers (v_cvt_scalef32_pk_bf16_fp8
//     with scale 1); P accumulates the two stages of a 128-K scale block on
//     v_mfma_f32_16x16x32_bf16, then acc += P * w_scale[n/128, kb].
// ---------------------------------------------------------------------------
// One tile shape serves every T > 64: 64 rows x 256 columns, 8 waves, two
// 32 KB stages, so two workgroups (16 waves) share a CU.  Each stage holds
// 64 K of the rows' bf16 hi and lo halves (128 + 128 bytes per row) and of
// 256 W2 rows.  With the activation pair, a three-stage ring (96 KB) would
// leave one workgroup per CU; measured against it and against 128 x 256
// tiles of 8 waves with three 48 KB stages (one per CU), the two-workgroup
// form was fastest at every T tried: T = 1024 113 against 140 us, T = 4000
// 830 against 1030 us, T = 8192 with four hot experts 1677 against 1816 us
// (the 128 x 256 kernel), uniform routing at T = 8192 537 against 612 us.
// Sixteen resident waves hide the stage barrier and the operand reads that
// eight could not: with eight, the first wave of each SIMD finishes its
// stage early and waits at the barrier while the second runs alone.  Sixteen
// waves in one 128 x 256 workgroup (three 48 KB stages, a quarter fewer
// copied bytes per flop) lost too: T = 1024 107 against 145 us, uniform
// routing at T = 8192 542 against 590 us.

template <int WM, int WN, int MI, int NJ, int STAGES>
struct G2Tiled {
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = kWave * kWaves;
  static constexpr int BM = 16 * MI * WM;
  static constexpr int BN = 16 * NJ * WN;
  static_assert(16 * NJ <= kBlk && kBlk % (16 * NJ) == 0, "a wave's columns lie in one scale block");
  static constexpr int kNT = kH / BN;
  static_assert(kH % BN == 0, "column tiles");
  static constexpr int kAFrags = BM / 16;
  static constexpr int kAFragBytes = 4096;  // hi (two wide planes), then lo (two wide planes)
  static constexpr int kAPlanes = 4 * kAFrags;
  static constexpr int kBFrags = BN / 16;
  static constexpr int kBOff = kAFrags * kAFragBytes;
  static constexpr int kStageBytes = kBOff + kBFrags * 1024;
  static constexpr int kWscBytes = kTopK * WN * kNIBlk * 4;  // weight block scales of up to 8 experts (after the stages)
  static constexpr int kStages = STAGES;
  static_assert(kStages >= 2 && kStages <= 5, "pipeline depth");
  static constexpr int kSteps = kI / 64;  // stages per tile (two per scale block)
  static constexpr int kPlanes = kAPlanes + kBFrags;
  static_assert(kPlanes % kWaves == 0, "planes must split evenly over waves");
  static constexpr int kPlanesPerWave = kPlanes / kWaves;
  static constexpr int kGroupM = 4;
};

template <int WM, int WN, int MI, int NJ, int STAGES>
__global__ void __launch_bounds__(64 * WM * WN, 4)
gemm2_tiled_kernel(const uint16_t* __restrict__ act, const uint8_t* __restrict__ w2,
                   const float* __restrict__ w2_scale, const int32_t* __restrict__ expert_off,
                   float* __restrict__ down, int T) {
  using C = G2Tiled<WM, WN, MI, NJ, STAGES>;
  // One LDS object (see gemm1.hip): the stage ring, then the weight scales.
  __shared__ __attribute__((aligned(1024))) char lds[C::kStages * C::kStageBytes + C::kWscBytes];

  ExpertRows X;
  X.load(expert_off);
  // Experts of every token (every_token_experts): a fused tile takes row tile
  // mt of each of them (tokens 64 mt ..), runs its K loop over all of them in
  // expert order into one accumulator (GEMM1 folded the routing weights into
  // their rows) and writes the sum to the first one's rows.
  const uint32_t fused = every_token_experts(X, T);
  int mt, nt, e, row0, rows;
  uint32_t tile_exps;  // the experts whose K loops this tile runs, in order
  if (!fused) {
    const int mt_total = X.count_tiles(C::BM);
    const int t = xcd_tile(blockIdx.x, mt_total * C::kNT);
    if (t < 0) return;
    grouped_tile(X, t, C::BM, C::kNT, C::kGroupM, mt, nt);
    X.find_tile(mt, C::BM, e, row0, rows);
    tile_exps = 1u << e;
  } else {
    // XCD x = block % 8 takes the x-th eighth of the fused tiles (the long
    // ones) first, then the x-th eighth of the other experts' tiles.
    const int lane = threadIdx.x & (kWave - 1);
    ExpertRows Xs = X;
    if (lane < kELocal && ((fused >> lane) & 1u)) Xs.cnt = 0;
    const int frt = (T + C::BM - 1) / C::BM;  // fused row tiles
    const int nf = frt * C::kNT, ns = Xs.count_tiles(C::BM) * C::kNT;
    const int x = blockIdx.x % 8, l = blockIdx.x / 8;
    const int f0 = (int)((int64_t)x * nf / 8), f1 = (int)((int64_t)(x + 1) * nf / 8);
    const int s0 = (int)((int64_t)x * ns / 8), s1 = (int)((int64_t)(x + 1) * ns / 8);
    if (l < f1 - f0) {
      // L2 groups of kGroupM row tiles sweeping the column tiles, row tile fastest
      const int idx = f0 + l, per_group = C::kGroupM * C::kNT;
      const int g = idx / per_group, within = idx % per_group;
      const int size = min(C::kGroupM, frt - g * C::kGroupM);
      mt = g * C::kGroupM + within % size;
      nt = within / size;
      e = __builtin_ctz(fused);
      row0 = X.begin(e) + mt * C::BM;
      rows = min(C::BM, T - mt * C::BM);
      tile_exps = fused;
    } else if (l - (f1 - f0) < s1 - s0) {
      grouped_tile(Xs, s0 + l - (f1 - f0), C::BM, C::kNT, C::kGroupM, mt, nt);
      Xs.find_tile(mt, C::BM, e, row0, rows);
      tile_exps = 1u << e;
    } else {
      return;
    }
  }
  const int n_steps = __builtin_popcount(tile_exps) * C::kSteps;
  const int n0 = nt * C::BN;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x & (kWave - 1);
  const int lq = lane >> 4;
  const int lr = lane & 15;
  const int wm = wave / WN;
  const int wn = wave % WN;
  // MFMA operand slots: A rows in wide layout (chunks 2q, 2q+1), B rows narrow (chunk q)
  const int slot_a0 = wide_slot(lr, 2 * lq), slot_a1 = wide_slot(lr, 2 * lq + 1), slot_b = narrow_slot(lr, lq);

  // DMA sources as a wave-uniform base (the tile's first act row, its first
  // W2 row) plus a 32-bit lane offset, one VGPR per plane, and LDS
  // destinations.  A plane 4f + 2h + p: rows 8p .. 8p+7 of row block f, hi
  // (h = 0) or lo (h = 1) half of the stage's 64 columns (128 bytes each,
  // adjacent in the act row).  Plane k of every wave is an A plane for k <
  // kAK, a B plane otherwise.  The stage's step goes into the 32-bit offset:
  // a 64-bit per-lane pointer took two VGPRs per plane (T = 8192: GEMM2
  // 1,646 -> 1,631 us, 128 -> 122 VGPRs).
  static_assert(C::kAPlanes % C::kWaves == 0, "plane k of every wave is of one kind");
  constexpr int kAK = C::kAPlanes / C::kWaves;
  // copy sources of the expert being copied: its act rows and W2 rows
  const char* abase = (const char*)(act + (size_t)row0 * kActRowElems);
  const char* bbase = (const char*)(w2 + ((size_t)e * kH + n0) * kI);
  int copy_exp = 0;  // its index in tile_exps
  uint32_t off[C::kPlanesPerWave];
  int dst[C::kPlanesPerWave];
#pragma unroll
  for (int k = 0; k < C::kPlanesPerWave; ++k) {
    const int plane = wave + k * C::kWaves;
    if (k < kAK) {
      const int f = plane >> 2, h = (plane >> 1) & 1, p = plane & 1;
      int fr, chunk;
      wide_copy_lane(lane, p, fr, chunk);
      const int r = min(f * 16 + fr, rows - 1);
      off[k] = (uint32_t)r * (kActRowElems * 2) + 128 * h + 16 * chunk;
      dst[k] = f * C::kAFragBytes + h * 2048 + p * 1024;
    } else {
      const int f = plane - C::kAPlanes;
      int fr, chunk;
      narrow_copy_lane(lane, fr, chunk);
      off[k] = (uint32_t)(16 * f + fr) * kI + 16 * chunk;
      dst[k] = C::kBOff + f * 1024;
    }
  }
  auto issue = [&](int s) {
    if (s / C::kSteps != copy_exp) {  // a fused tile's next expert (wave-uniform)
      copy_exp = s / C::kSteps;
      uint32_t m = tile_exps;
      for (int k = 0; k < copy_exp; ++k) m &= m - 1;
      const int d = __builtin_ctz(m);
      abase = (const char*)(act + (size_t)(expert_off[d] + mt * C::BM) * kActRowElems);
      bbase = (const char*)(w2 + ((size_t)d * kH + n0) * kI);
    }
    // the buffer of global step s is s % kStages, as step() reads it
    static_assert(C::kSteps % C::kStages == 0, "an expert's step count keeps the ring position");
    s %= C::kSteps;
    char* base = lds + (s % C::kStages) * C::kStageBytes;
    // bytes per stage: bf16 hi + lo A, e4m3 B; A row blocks wholly past the
    // tile's rows are never read: no copy
#pragma unroll
    for (int k = 0; k < C::kPlanesPerWave; ++k) {
      if (k < kAK) {
        if (((wave + k * C::kWaves) >> 2) * 16 < rows) dma16(abase + (uint32_t)(s * 256 + off[k]), base + dst[k]);
      } else {
        dma16(bbase + (uint32_t)(s * 64 + off[k]), base + dst[k]);
      }
    }
  };
  // weight block scales of every wave's columns, staged in LDS once
  float* wsc = (float*)(lds + C::kStages * C::kStageBytes);  // [expert of the tile][WN][16]
  for (int i = threadIdx.x; i < n_steps / C::kSteps * WN * kNIBlk; i += C::kThreads) {
    const int di = i / (WN * kNIBlk), w_n = (i / kNIBlk) % WN, kb = i % kNIBlk;
    uint32_t m = tile_exps;
    for (int k = 0; k < di; ++k) m &= m - 1;
    wsc[i] = w2_scale[((size_t)__builtin_ctz(m) * kNHBlk + (n0 + 16 * NJ * w_n) / kBlk) * kNIBlk + kb];
  }

  v4f acc[MI][NJ], P[MI][NJ];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) acc[mi][nj] = v4f{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int s = 0; s < C::kStages - 1; ++s) issue(s);
  // Two steps (one 128-K weight scale block) per iteration: the block's
  // first MFMAs start from a zero accumulator, the second step's results are
  // scaled into acc.
  static_assert(C::kSteps % 2 == 0, "steps pair into scale blocks");
  static_assert(C::kStages == 2, "skipped copies leave the per-stage counts unequal: every wait is for all");
  auto step = [&](int s, bool first, auto live_c) {
    constexpr int L = decltype(live_c)::value;  // live 16-row blocks of this wave
    // stages s+1 .. s+kStages-2 may stay in flight
    wait_stages_ahead<C::kPlanesPerWave>(min(n_steps - 1 - s, C::kStages - 2));
    block_barrier();
    if (s + C::kStages - 1 < n_steps) issue(s + C::kStages - 1);

    const char* sbuf = lds + (s % C::kStages) * C::kStageBytes;
    v8bf a[MI][2], al[MI][2], b[NJ][2];
#pragma unroll
    for (int mi = 0; mi < L; ++mi) {
      const char* f = sbuf + (wm * MI + mi) * C::kAFragBytes;
      a[mi][0] = *(const v8bf*)(f + slot_a0);
      a[mi][1] = *(const v8bf*)(f + slot_a1);
      al[mi][0] = *(const v8bf*)(f + 2048 + slot_a0);
      al[mi][1] = *(const v8bf*)(f + 2048 + slot_a1);
    }
#pragma unroll
    for (int nj = 0; nj < (L > 0 ? NJ : 0); ++nj) {
      const v4i raw = *(const v4i*)(sbuf + C::kBOff + (wn * NJ + nj) * 1024 + slot_b);
      b[nj][0] = e4m3x8_to_bf16((uint32_t)raw[0], (uint32_t)raw[1]);
      b[nj][1] = e4m3x8_to_bf16((uint32_t)raw[2], (uint32_t)raw[3]);
    }
#pragma unroll
    for (int mi = 0; mi < L; ++mi)
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj) {
        P[mi][nj] = mfma_bf16_16x16x32(a[mi][0], b[nj][0], first ? v4f{0.f, 0.f, 0.f, 0.f} : P[mi][nj]);
        P[mi][nj] = mfma_bf16_16x16x32(a[mi][1], b[nj][1], P[mi][nj]);
        P[mi][nj] = mfma_bf16_16x16x32(al[mi][0], b[nj][0], P[mi][nj]);
        P[mi][nj] = mfma_bf16_16x16x32(al[mi][1], b[nj][1], P[mi][nj]);
      }
    if (!first) {
      const float sb = wsc[(s / C::kSteps * WN + wn) * kNIBlk + ((s % C::kSteps) >> 1)];
#pragma unroll
      for (int mi = 0; mi < L; ++mi)
#pragma unroll
        for (int nj = 0; nj < NJ; ++nj)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[mi][nj][i] = __builtin_fmaf(P[mi][nj][i], sb, acc[mi][nj][i]);
    }
  };
  // Row blocks past the tile's rows (experts with few rows) are neither
  // copied nor multiplied; the choice is per wave and per tile, so each count
  // of live blocks gets its own loop (T = 65: GEMM2 53.8 -> 44.7 us, T = 256
  // 69.8 -> 60.9 us; T = 8192 unchanged).  The three loops would take 132
  // VGPRs; the launch bounds hold them to the 128 that keep two workgroups
  // per CU, without spills.
  auto run = [&](auto live_c) {
#pragma unroll 1
    for (int s = 0; s < n_steps; s += 2) {
      step(s, true, live_c);
      step(s + 1, false, live_c);
    }
  };
  const int live = min(MI, max(0, (rows - wm * MI * 16 + 15) / 16));
  static_assert(MI == 2, "live-block loops for MI = 2");
  if (live == MI)
    run(std::integral_constant<int, MI>{});
  else if (live == 1)
    run(std::integral_constant<int, 1>{});
  else
    run(std::integral_constant<int, 0>{});

#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = (wm * MI + mi) * 16 + 4 * lq + i;
        if (r < rows) down[(size_t)(row0 + r) * kH + n0 + 16 * (wn * NJ + nj) + lr] = acc[mi][nj][i];
      }
}

template <int WM, int WN, int MI, int NJ, int STAGES>
hipError_t launch_gemm2_tiled(int T, const uint8_t* w2, const float* w2_scale, const Layout& L, char* ws,
                              hipStream_t stream) {
  using C = G2Tiled<WM, WN, MI, NJ, STAGES>;
  const int64_t pairs = (int64_t)T * kTopK;
  const int64_t mtiles = (pairs + C::BM - 1) / C::BM + (pairs < kELocal ? pairs : kELocal);
  const int64_t blocks = ((mtiles * C::kNT + 7) / 8) * 8;
  hipLaunchKernelGGL((gemm2_tiled_kernel<WM, WN, MI, NJ, STAGES>), dim3((unsigned)blocks), dim3(C::kThreads), 0,
                     stream, (const uint16_t*)(ws + L.act), w2, w2_scale,
                     (const int32_t*)(ws + L.expert_off), (float*)(ws + L.down), T);
  return hipGetLastError();
}

}  // namespace

bool gemm2_fuses_combine(int T) { return T <= kGemm2StreamMaxTokens; }

hipError_t launch_gemm2(int T, const uint8_t* w2, const float* w2_scale, const Layout& L, char* ws, void* out,
                        hipStream_t stream) {
  if (gemm2_fuses_combine(T)) {
    hipLaunchKernelGGL(gemm2_combine_kernel, dim3(kS2Units), dim3(kS2Threads), 0, stream,
                       (const uint16_t*)(ws + L.act), w2, w2_scale, (const int32_t*)(ws + L.expert_off),
                       (const int32_t*)(ws + L.perm_token), (const float*)(ws + L.perm_w), T, (uint16_t*)out);
    return hipGetLastError();
  }
  return launch_gemm2_tiled<2, 4, 2, 4, 2>(T, w2, w2_scale, L, ws, stream);
}

}  // namespace moe
