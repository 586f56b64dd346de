// moe_common.hpp -- shared constants, workspace layout and device helpers of
// the gfx950 FP8 block-scale MoE layer.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <stddef.h>
#include <stdint.h>

namespace moe {

// Geometry fixed by the definition (moe.py:65-76; moe.cu:39-51).
constexpr int kH = 7168;          // hidden size
constexpr int kI = 2048;          // intermediate size
constexpr int k2I = 4096;         // gate + up
constexpr int kELocal = 32;       // local experts
constexpr int kEGlobal = 256;     // global experts
constexpr int kTopK = 8;
constexpr int kNGroup = 8;
constexpr int kTopKGroup = 4;
constexpr int kGroupSize = 32;
constexpr int kBlk = 128;         // quantisation block
constexpr int kNHBlk = kH / kBlk;   // 56
constexpr int kNIBlk = kI / kBlk;   // 16
constexpr int kN2IBlk = k2I / kBlk; // 32
constexpr int kWave = 64;

// Largest T any entry point accepts.  Every row index (< 8T) and grid
// dimension stays inside int32, and every byte offset of a token row inside
// hidden_states (token * 7168 + 7167) inside uint32: the wide GEMM1 builds
// its copy addresses as a wave-uniform base plus a 32-bit lane offset, which
// would wrap from token 599,187 (2^32 / 7168) on.
constexpr int64_t kMaxTokens = 1 << 19;
static_assert(kMaxTokens * kH <= (int64_t)1 << 32, "token row offsets fit in 32 bits");

// Largest T for which GEMM2 also performs the weighted combine: its rows
// never reach the workspace, and no combine pass runs.
constexpr int kGemm2StreamMaxTokens = 64;
// From this T on, experts that every token selects are summed inside GEMM2
// (every_token_experts).  Below it the fused tiles (T / 64 row tiles x 28
// column tiles, each running several experts' K loops) are too few to fill
// the chip's 512 workgroup slots: four such experts, interleaved A/B, layer
// us (unfused -> fused): T = 640 356 -> 388, 896 424 -> 425, 1152 553 -> 542,
// 2048 814 -> 772, 8192 2849 -> 2712.
constexpr int kEveryTokenFuseMinTokens = 1024;

// SwiGLU activation rows (`act`) hold each fp32 value v as a pair of bf16,
// hi = bf16(v) and lo = bf16(v - hi), so hi + lo carries v to ~2^-17
// relative: GEMM2 multiplies both on bf16 MFMA, as the fp32 activation of the
// reference (moe.py:190-196) needs -- a single bf16 rounding leaves the
// output within 1e-2 only while its magnitude stays small.  A row is 32
// chunks of 64 columns, chunk c = [hi of columns 64c..64c+63][lo of the
// same], 8 KB per row: one 64-column step of GEMM2 reads 256 contiguous bytes
// per row.
constexpr int kActRowElems = 2 * kI;  // bf16 elements per act row
// Element index of the hi half of column `col` inside an act row (lo at +64).
__host__ __device__ constexpr int act_col(int col) { return (col >> 6) * 128 + (col & 63); }

struct Layout {
  size_t topk_ids, topk_w, pair_row, expert_off, perm_token, perm_w, act, down, block_hist, total;
};

constexpr size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

constexpr Layout make_layout(int64_t T) {
  Layout L{};
  size_t off = 0;
  auto take = [&off](size_t bytes) {
    const size_t at = off;
    off = align_up(off + bytes, 256);
    return at;
  };
  const size_t rows = (size_t)T * kTopK;  // upper bound on routed local pairs
  L.expert_off = take(64 * sizeof(int32_t));
  L.topk_ids = take(rows * sizeof(int32_t));
  L.topk_w = take(rows * sizeof(float));
  L.pair_row = take(rows * sizeof(int32_t));
  L.perm_token = take(rows * sizeof(int32_t));
  L.perm_w = take(rows * sizeof(float));
  L.act = take(rows * kActRowElems * sizeof(uint16_t));
  // fp32 GEMM2 rows, only where a separate combine pass reads them
  L.down = take(T > kGemm2StreamMaxTokens ? rows * kH * sizeof(float) : 0);
  L.block_hist = take((size_t)((T + 3) / 4) * kELocal * sizeof(int32_t));  // per route workgroup (4 tokens)
  L.total = off;
  return L;
}

// ---------------------------------------------------------------------------
// LDS operand tiles.  A 16-row MFMA fragment is staged in LDS row-major:
//   * wide: 128 bytes of K per row, two 1 KB planes of 8 rows each;
//   * narrow: 64 bytes of K per row, one 1 KB plane of 16 rows.
// Tiles are copied global -> LDS with global_load_lds_dwordx4, where lane i
// of a copy always writes bytes 16i .. 16i+15 of its plane.  Lane i is given
// the (row, 16-byte chunk) that makes
//   * 8 (wide) or 4 (narrow) consecutive lanes read one row's 128 or 64
//     contiguous bytes -- the vector memory path coalesces consecutive lanes,
//     and a copy whose consecutive lanes touch different rows runs at about
//     half the L2 -> LDS rate;
//   * chunk c of row r land at slot c ^ swz(r), so that the MFMA operand
//     reads, where the 16 lanes of a quarter read 16 rows at the same logical
//     chunk, fall on distinct 16-byte bank groups both within every 8 lanes
//     (128 bytes of banks) and within all 16 (256 bytes).  The narrow
//     swizzle (r/4 ^ r/2) is the one that satisfies both: r/4 alone left
//     GEMM2's B reads with bank conflicts on a third of the LDS cycles.
// MFMA lane (q = lane / 16, r = lane % 16) reads row r at logical chunks
//   * wide: 2q and 2q + 1 (K bytes 32q .. 32q+31 of the row);
//   * narrow: q (K bytes 16q .. 16q+15).
// Both operands of an MFMA use the same mapping, so K is in natural order and
// the bf16 activation rows are stored in natural column order.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int swz_wide(int r) { return (r & 7) ^ (r >> 3); }  // r < 16
__device__ __forceinline__ int swz_narrow(int r) { return ((r >> 2) ^ (r >> 1)) & 3; }  // r < 16

// Copy lane -> (row of the fragment, source chunk) for wide plane `half`.
__device__ __forceinline__ void wide_copy_lane(int lane, int half, int& row, int& chunk) {
  row = 8 * half + (lane >> 3);
  chunk = (lane & 7) ^ swz_wide(row);
}
// Copy lane -> (row, source chunk) for a narrow plane.
__device__ __forceinline__ void narrow_copy_lane(int lane, int& row, int& chunk) {
  row = lane >> 2;
  chunk = (lane & 3) ^ swz_narrow(row);
}
// Byte offset of (row r, logical chunk c) inside a wide fragment / narrow plane.
__device__ __forceinline__ int wide_slot(int r, int c) { return 1024 * (r >> 3) + 128 * (r & 7) + 16 * (c ^ swz_wide(r)); }
__device__ __forceinline__ int narrow_slot(int r, int c) { return 64 * r + 16 * (c ^ swz_narrow(r)); }

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// fp32 -> bf16 bits, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }

typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf_t __attribute__((ext_vector_type(2)));

// (a, b) -> bf16 bits a | b << 16, both rounded to nearest even, in one
// v_cvt_pk_bf16_f32 (equal to f32_to_bf16_rne for every fp32 but NaN payloads;
// checked exhaustively by the test suite).
__device__ __forceinline__ uint32_t bf16x2_rne(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{a, b}, v2bf_t));
}

// Two values -> their (hi, lo) bf16 pairs, packed as bf16x2_rne packs:
// hi = RNE(v), lo = RNE(v - hi); v - hi is exact in fp32.  A non-finite hi
// keeps lo = 0, so hi + lo stays inf / NaN like v.
__device__ __forceinline__ void split_bf16x2(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = bf16x2_rne(a, b);
  const float ha = __uint_as_float(hi << 16), hb = __uint_as_float(hi & 0xFFFF0000u);
  lo = bf16x2_rne(__builtin_isfinite(ha) ? a - ha : 0.f, __builtin_isfinite(hb) ? b - hb : 0.f);
}

// One value -> its (hi, lo) bf16 pair.
__device__ __forceinline__ void split_bf16(float v, uint16_t& hi, uint16_t& lo) {
  uint32_t h, l;
  split_bf16x2(v, 0.f, h, l);
  hi = (uint16_t)h;
  lo = (uint16_t)l;
}

// SwiGLU of one (gate x1, up x2) pair: silu(x2) * x1 = x2 / (1 + e^-x2) * x1
// (moe.py:190-193), with the hardware exp2 and reciprocal (v_exp_f32,
// v_rcp_f32: ~1 ulp each) in place of correctly rounded division: a few ulp
// against the reference's fp32 ops, far below the ~1e-5 relative error the
// fp8 MFMA block sums already carry into x1 and x2.  x2 -> -inf gives -0 as
// the reference does (e^-x2 = inf, rcp = 0).
__device__ __forceinline__ float silu_mul(float x2, float x1) {
  const float e = __builtin_amdgcn_exp2f(-x2 * 1.44269504088896341f);
  return x2 * __builtin_amdgcn_rcpf(1.0f + e) * x1;
}

// Order-preserving map of a (non-NaN) float to uint32.
__device__ __forceinline__ uint32_t float_order_key(float v) {
  uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float float_from_order_key(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  lo = __shfl_xor(lo, mask, kWave);
  hi = __shfl_xor(hi, mask, kWave);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t u64max(uint64_t a, uint64_t b) { return a > b ? a : b; }

// D = A(16x128 e4m3) * B(128x16 e4m3), fp32 16x16 result (no accumulate-in).
// Lane l supplies 32 K-bytes of row (l % 16) of A and of column (l % 16) of
// B; lanes l/16 = 0..3 cover the four 32-byte quarters of the 128 K values.
// Output: lane l holds rows 4*(l/16)+i, column l % 16, i = 0..3.
__device__ __forceinline__ v4f mfma_f8_16x16x128(const v8i& a, const v8i& b) {
  v4f z = {0.f, 0.f, 0.f, 0.f};
  // Format codes 0/0 = e4m3 for both operands; zero scale operands select
  // the unscaled v_mfma_f32_16x16x128_f8f6f4.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 0, 0, 0);
}

// D = C + A(16x32 bf16) * B(32x16 bf16): lane l supplies 8 K-values of row
// (l % 16) of A / column (l % 16) of B at K = 8*(l/16) .. +8.
__device__ __forceinline__ v4f mfma_bf16_16x16x32(const v8bf& a, const v8bf& b, const v4f& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 8 e4m3 bytes (two dwords) -> 8 bf16 (exact: every e4m3 value is a bf16).
__device__ __forceinline__ v8bf e4m3x8_to_bf16(uint32_t lo, uint32_t hi) {
  v2bf p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
  v2bf p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
  v2bf p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
  v2bf p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
  v8bf r;
  r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
  r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
  return r;
}

// ---------------------------------------------------------------------------
// LDS staging helpers
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void;

// Asynchronous global -> LDS copy (global_load_lds_dwordx4): lane i writes its
// 16 bytes at lds_wave_base + 16 * i.  lds_wave_base must be wave-uniform.
__device__ __forceinline__ void dma16(const void* g, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_wave_base, 16, 0, 0);
}
// Same with the nontemporal (nt) cache policy, for data read exactly once:
// the streaming kernels' expert weights (small_t64: GEMM1 101 -> 87 us).  The
// tiled kernels re-read weight tiles through L2 and keep dma16 (nt there made
// GEMM2 at T = 8192 34% slower).
__device__ __forceinline__ void dma16_nt(const void* g, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_wave_base, 16, 0, 2);
}
// Same with 4 bytes per lane (global_load_lds_dword): lane i -> base + 4 * i.
__device__ __forceinline__ void dma4(const void* g, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_wave_base, 4, 0, 0);
}

// s_waitcnt vmcnt(N) lgkmcnt(0): at most N vector-memory operations of this
// wave (loads and LDS DMA, completed in issue order) still outstanding, and
// every LDS access of this wave complete.
template <int N>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (0 << 8));
}

// s_waitcnt vmcnt(N) alone (lgkmcnt left at its maximum): scalar and LDS
// loads may stay in flight.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Waits until at most `ahead` pipeline stages of `per_stage` vector-memory
// operations each are still in flight (ahead = 0, 1, 2, 3).
template <int per_stage>
__device__ __forceinline__ void wait_stages_ahead(int ahead) {
  if (ahead >= 5)
    wait_vmcnt_lgkm0<5 * per_stage>();
  else if (ahead == 4)
    wait_vmcnt_lgkm0<4 * per_stage>();
  else if (ahead == 3)
    wait_vmcnt_lgkm0<3 * per_stage>();
  else if (ahead == 2)
    wait_vmcnt_lgkm0<2 * per_stage>();
  else if (ahead == 1)
    wait_vmcnt_lgkm0<per_stage>();
  else
    wait_vmcnt_lgkm0<0>();
}

// s_waitcnt vmcnt(n) lgkmcnt(0) for a wave-uniform runtime n in [0, 8]
// (larger n waits for n = 8).
__device__ __forceinline__ void wait_vmcnt_lgkm0_rt(int n) {
  switch (n) {
    case 0: wait_vmcnt_lgkm0<0>(); break;
    case 1: wait_vmcnt_lgkm0<1>(); break;
    case 2: wait_vmcnt_lgkm0<2>(); break;
    case 3: wait_vmcnt_lgkm0<3>(); break;
    case 4: wait_vmcnt_lgkm0<4>(); break;
    case 5: wait_vmcnt_lgkm0<5>(); break;
    case 6: wait_vmcnt_lgkm0<6>(); break;
    case 7: wait_vmcnt_lgkm0<7>(); break;
    default: wait_vmcnt_lgkm0<8>(); break;
  }
}

// ---- DPP helpers (GFX9 controls) -------------------------------------------
constexpr int kDppQuad1032 = 0xB1;    // quad_perm [1,0,3,2]
constexpr int kDppQuad2301 = 0x4E;    // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowBcast15 = 0x142;

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  if constexpr (ROW_MASK == 0xF) {
    // every lane reads a lane of its own row (quad permutes, row mirrors):
    // a bound_ctrl move, which the compiler folds into the consuming VALU op
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
  } else {
    // lanes outside ROW_MASK keep their own value (old = v)
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, ROW_MASK, 0xF, false);
  }
}

// Maximum of a 32-bit value over each row of 16 lanes, in every lane of the row.
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t k) {
  k = max(k, dpp_u32<kDppQuad1032, 0xF>(k));
  k = max(k, dpp_u32<kDppQuad2301, 0xF>(k));
  k = max(k, dpp_u32<kDppRowHalfMirror, 0xF>(k));
  k = max(k, dpp_u32<kDppRowMirror, 0xF>(k));
  return k;
}

// Workgroup barrier that the compiler may not move memory accesses across.
__device__ __forceinline__ void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Workgroup barrier for LDS hand-offs only: this wave's LDS accesses are
// complete, its vector-memory loads and copies may still be in flight
// (__syncthreads would wait for those too).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// XCD-aware block -> tile map.  Workgroups are dispatched round-robin over the
// 8 XCDs (block b runs on XCD b % 8), so block b takes tile
//   (b % 8) * ceil(R / 8) + b / 8
// of the R real tiles: each XCD walks one contiguous run of the tile order,
// and tiles that share operands share that XCD's L2.  Returns -1 for blocks
// past the real tiles.
__device__ __forceinline__ int xcd_tile(int b, int R) {
  const int per = (R + 7) / 8;
  const int t = (b % 8) * per + b / 8;
  return (b < per * 8 && t < R) ? t : -1;
}

// Workgroups of one kernel that fit on the current device at once (compute
// units x resident workgroups per CU), queried on the first launch on each
// device (a process may drive devices of different sizes).  A persistent
// kernel launches min(work items, this) workgroups and strides over its
// items.
struct ResidentGrid {
  static constexpr int kMaxDevices = 64;
  const void* kernel;
  int threads;
  size_t dyn_lds;
  std::atomic<int> n[kMaxDevices] = {};
  template <typename Kernel>
  ResidentGrid(Kernel k, int t, size_t lds = 0) : kernel((const void*)k), threads(t), dyn_lds(lds) {}
  int count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = 0;
    int v = n[dev].load(std::memory_order_relaxed);
    if (v <= 0) {
      int cus = 0, per = 0;
      if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
          hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, dyn_lds) == hipSuccess)
        v = cus * (per > 0 ? per : 1);
      if (v <= 0) v = 256;
      n[dev].store(v, std::memory_order_relaxed);  // every thread computes the same value
    }
    return v;
  }
  int limit(int items) {
    const int c = count();
    return items < c ? (items > 0 ? items : 1) : c;
  }
};

// Index of the k-th set bit of m (k < popcount(m)).
__device__ __forceinline__ int nth_set_bit(uint32_t m, int k) {
  for (int i = 0; i < k; ++i) m &= m - 1;
  return __builtin_ctz(m);
}

// Persistent form of xcd_tile: a grid of G workgroups (a multiple of 8) over
// R tiles.  XCD x = b % 8 still owns the tile range [x * per, (x + 1) * per);
// its G / 8 workgroups take the range's tiles round robin, so at any time an
// XCD's workgroups work on neighbouring tiles.  The i-th tile of workgroup b,
// or -1 past the last.
__device__ __forceinline__ int xcd_tile_nth(int b, int G, int R, int i) {
  const int per = (R + 7) / 8;
  const int l = b / 8 + i * (G / 8);
  const int t = (b % 8) * per + l;
  return (l < per && t < R) ? t : -1;
}

// The 33 expert row offsets spread over the lanes of a wave (lane x holds
// off[x], lanes past 32 hold off[32]), read with one vector load.  Every query
// is wave-level (ballot / readlane / lane scan): all 64 lanes of the wave must
// call it, and the results are wave-uniform.
struct ExpertRows {
  int o;    // off[min(lane, 32)]
  int cnt;  // rows of expert `lane` (lanes < 32), else 0

  __device__ __forceinline__ void load(const int32_t* __restrict__ off) {
    const int lane = threadIdx.x & (kWave - 1);
    o = off[min(lane, kELocal)];
    const int o1 = __shfl_down(o, 1, kWave);
    cnt = lane < kELocal ? o1 - o : 0;
  }
  __device__ __forceinline__ int begin(int e) const { return __builtin_amdgcn_readlane(o, e); }
  __device__ __forceinline__ int end(int e) const { return __builtin_amdgcn_readlane(o, e + 1); }
  // Bit e set <=> expert e has rows.
  __device__ __forceinline__ uint32_t active() const { return (uint32_t)__ballot(cnt > 0); }
  // The slot-th expert with rows, or -1.
  __device__ __forceinline__ int nth_active(int slot) const {
    uint32_t m = active();
    for (int k = 0; k < slot && m; ++k) m &= m - 1;
    return m ? __builtin_ctz(m) : -1;
  }
  // Inclusive scan over experts of the number of row tiles of height bm.
  __device__ __forceinline__ int tiles_incl(int bm) const {
    const int lane = threadIdx.x & (kWave - 1);
    const int nt = (cnt + bm - 1) / bm;
    int incl = nt;
#pragma unroll
    for (int d = 1; d < kELocal; d <<= 1) {
      const int v = __shfl_up(incl, d, kWave);
      if (lane >= d) incl += v;
    }
    return incl;
  }
  __device__ __forceinline__ int count_tiles(int bm) const {
    return __builtin_amdgcn_readlane(tiles_incl(bm), kELocal - 1);
  }
  // The L2 group of global row tile `tile` (< count_tiles(bm)): the run of at
  // most gm row tiles of one expert that holds it; each expert's runs start
  // at its first row tile.
  __device__ __forceinline__ void tile_group(int tile, int bm, int gm, int& first, int& size) const {
    const int lane = threadIdx.x & (kWave - 1);
    const int incl = tiles_incl(bm);
    const uint64_t m = __ballot(lane < kELocal && incl > tile);
    const int e = m ? __builtin_ctzll(m) : kELocal - 1;
    const int e_end = __builtin_amdgcn_readlane(incl, e);
    const int e_begin = e_end - __builtin_amdgcn_readlane((cnt + bm - 1) / bm, e);
    first = e_begin + (tile - e_begin) / gm * gm;
    size = min(gm, e_end - first);
  }
  // Global row tile `tile` -> (expert, first row, rows in tile); false past the
  // last tile.
  __device__ __forceinline__ bool find_tile(int tile, int bm, int& e, int& row0, int& rows) const {
    const int lane = threadIdx.x & (kWave - 1);
    const int incl = tiles_incl(bm);
    const uint64_t m = __ballot(lane < kELocal && incl > tile);
    if (!m) return false;
    e = __builtin_ctzll(m);
    const int nt = (cnt + bm - 1) / bm;
    const int excl = __builtin_amdgcn_readlane(incl - nt, e);
    row0 = begin(e) + (tile - excl) * bm;
    rows = min(bm, end(e) - row0);
    return true;
  }
};

// Local experts that all T tokens select (T rows each, row begin + t being
// token t), as a bit mask, when at least two do and T >=
// kEveryTokenFuseMinTokens; else 0.  Their GEMM2 rows are summed per token inside
// GEMM2 instead of in the combine: GEMM1 scales their SwiGLU rows by the
// routing weights, a fused GEMM2 tile runs the K loop of every such expert
// into one accumulator and writes the sum to the first one's rows, and the
// combine adds that row once, at the first one's place in expert order.  At
// most 8 experts (N_sel <= 8 T).  Wave-level; every kernel of a call gets the
// same mask.
__device__ __forceinline__ uint32_t every_token_experts(const ExpertRows& X, int T) {
  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t m = (uint32_t)__ballot(lane < kELocal && X.cnt == T);
  static_assert(kEveryTokenFuseMinTokens > kGemm2StreamMaxTokens, "fused experts need the combine pass");
  return (T >= kEveryTokenFuseMinTokens && __builtin_popcount(m) >= 2) ? m : 0u;
}

// The local expert whose rows hold permuted row r (< N_sel).  Wave-level.
__device__ __forceinline__ int expert_of_row(const ExpertRows& X, int r) {
  const int lane = threadIdx.x & (kWave - 1);
  return __popcll(__ballot(lane < kELocal && X.o <= r)) - 1;
}

// Tile order inside the run: each L2 group (ExpertRows::tile_group) sweeps
// all `nt` column tiles, row tile fastest, so concurrently running blocks
// reuse the weight columns of their expert and the rows of their row tile.
// A group covers tiles [first * nt, (first + size) * nt), so the row tile
// t / nt lies in the group of tile t.
__device__ __forceinline__ void grouped_tile(const ExpertRows& X, int t, int bm, int nt, int gm, int& mt,
                                             int& ntile) {
  int first, size;
  X.tile_group(t / nt, bm, gm, first, size);
  const int r = t - first * nt;
  mt = first + r % size;
  ntile = r / size;
}

// Inclusive sum of v over lanes 0 .. lane (all 64 lanes take part).
__device__ __forceinline__ int lane_scan_incl(int v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int u = __shfl_up(v, d, kWave);
    if (lane >= d) v += u;
  }
  return v;
}

// Tile map that gives each of the 8 XCDs one eighth of every expert's tiles.
// Each expert's n_e = nt * (row tiles) tiles are taken in the order of
// grouped_tile (L2 groups of at most gm row tiles sweeping the nt column
// tiles); XCD x owns the contiguous slice [x n_e / 8, (x + 1) n_e / 8) of each
// expert, and its l-th tile is found by walking its slices in expert order.
// Against contiguous eighths of the whole tile order (xcd_tile), where one
// XCD could hold nothing but a hot expert's full tiles while another held the
// short tiles of small experts, every XCD now gets the same mix; a hot
// expert's L2 groups still stay whole on one XCD.  Wave-level; false past
// the XCD's last tile.
__device__ __forceinline__ bool xcd_expert_tile(const ExpertRows& X, int x, int l, int bm, int nt, int gm, int& mt,
                                                int& ntile) {
  const int lane = threadIdx.x & (kWave - 1);
  const int rt = (X.cnt + bm - 1) / bm;  // lane e < 32: row tiles of expert e (0 elsewhere)
  const int n = rt * nt;                  // its tiles
  const int lo = (int)(((int64_t)x * n) / 8), hi = (int)(((int64_t)(x + 1) * n) / 8);
  const int size = hi - lo;               // its slice on XCD x
  const int incl = lane_scan_incl(size);
  if (l >= __builtin_amdgcn_readlane(incl, kWave - 1)) return false;
  const int e = __builtin_ctzll(__ballot(incl > l));
  const int i = __builtin_amdgcn_readlane(lo, e) + l - (__builtin_amdgcn_readlane(incl, e) - __builtin_amdgcn_readlane(size, e));
  const int rte = __builtin_amdgcn_readlane(rt, e);
  const int tb = __builtin_amdgcn_readlane(lane_scan_incl(rt) - rt, e);  // row tiles before expert e
  // expert-local index i -> (row tile, column tile) in grouped_tile's order
  const int ng = (rte + gm - 1) / gm;
  const int j = min(i / (gm * nt), ng - 1);
  const int o = i - j * gm * nt;
  const int rows_g = min(gm, rte - j * gm);
  mt = tb + j * gm + o % rows_g;
  ntile = o / rows_g;
  return true;
}

// Row tiles of two heights: an expert's row tiles hold bm rows, its last one
// fewer; a last row tile of at most bm / 2 rows is "short", every other row
// tile "tall".  Totals over the experts (wave-level, uniform results).
__device__ __forceinline__ void tall_short_row_tiles(const ExpertRows& X, int bm, int& n_tall, int& n_short) {
  const int rt = (X.cnt + bm - 1) / bm;  // lane e < 32: row tiles of expert e
  const int sh = rt > 0 && X.cnt - (rt - 1) * bm <= bm / 2 ? 1 : 0;
  n_short = __builtin_amdgcn_readlane(lane_scan_incl(sh), kWave - 1);
  n_tall = __builtin_amdgcn_readlane(lane_scan_incl(rt), kWave - 1) - n_short;
}

// Tile map for those two heights.  XCD x takes an eighth of every expert's
// tall tiles and an eighth of its short tiles (as xcd_expert_tile does for one
// height); its list holds all its tall tiles (expert order, grouped_tile order
// inside an expert) before its short ones, so that the longer tiles start
// first.  mt is the row tile in ExpertRows::find_tile(mt, bm) numbering.
// Wave-level; false past the XCD's last tile.
__device__ __forceinline__ bool xcd_tall_first_tile(const ExpertRows& X, int x, int l, int bm, int nt, int gm,
                                                    int& mt, int& ntile) {
  const int rt = (X.cnt + bm - 1) / bm;
  const int sh = rt > 0 && X.cnt - (rt - 1) * bm <= bm / 2 ? 1 : 0;  // its last row tile is short
  const int tall = rt - sh;
  const int tb = lane_scan_incl(rt) - rt;  // row tiles before expert e
  {
    const int n = tall * nt;
    const int lo = (int)(((int64_t)x * n) / 8), hi = (int)(((int64_t)(x + 1) * n) / 8);
    const int size = hi - lo;
    const int incl = lane_scan_incl(size);
    const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
    if (l < total) {
      const int e = __builtin_ctzll(__ballot(incl > l));
      const int i = __builtin_amdgcn_readlane(lo, e) + l -
                    (__builtin_amdgcn_readlane(incl, e) - __builtin_amdgcn_readlane(size, e));
      const int rte = __builtin_amdgcn_readlane(tall, e);
      const int ng = (rte + gm - 1) / gm;
      const int j = min(i / (gm * nt), ng - 1);
      const int o = i - j * gm * nt;
      const int rows_g = min(gm, rte - j * gm);
      mt = __builtin_amdgcn_readlane(tb, e) + j * gm + o % rows_g;
      ntile = o / rows_g;
      return true;
    }
    l -= total;
  }
  const int n = sh * nt;
  const int lo = (int)(((int64_t)x * n) / 8), hi = (int)(((int64_t)(x + 1) * n) / 8);
  const int size = hi - lo;
  const int incl = lane_scan_incl(size);
  if (l >= __builtin_amdgcn_readlane(incl, kWave - 1)) return false;
  const int e = __builtin_ctzll(__ballot(incl > l));
  ntile = __builtin_amdgcn_readlane(lo, e) + l -
          (__builtin_amdgcn_readlane(incl, e) - __builtin_amdgcn_readlane(size, e));
  mt = __builtin_amdgcn_readlane(tb, e) + __builtin_amdgcn_readlane(tall, e);  // the expert's last row tile
  return true;
}

}  // namespace moe
