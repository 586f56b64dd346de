// gemm1.hip -- grouped FP8 GEMM1 (hidden 7168 -> gate/up 4096) with the
// per-128-K block-scale dequantisation folded into the fp32 accumulator and
// SwiGLU fused into the epilogue; writes the bf16 activation rows GEMM2 reads.
//
// Reference behaviour: moe.py:186-193 (G1 = A_e W13_e^T; C = silu(G1[:, I:]) *
// G1[:, :I]); CUDA solution gemm_fp8_fp8_grouped_kernel (moe.cu:1373-1609) and
// swiglu_kernel (moe.cu:2125-2146), which round-trip G1 through fp32 HBM.
//
// Design (gfx950): v_mfma_f32_16x16x128_f8f6f4 covers exactly one 128-wide K
// scale block per instruction, so each MFMA yields the unscaled block partial P
// and the accumulator takes  acc += P * (a_scale[row, kb] * w_scale[n/128, kb]).
// fp8 x fp8 products are exact; only the fp32 summation order differs from the
// fp32 reference.  Gate column j and up column 2048 + j always land in the same
// lane (or in lanes r and r + 8), so SwiGLU is fused into the epilogue and G1
// never reaches HBM.  Two kernels:
//   * streaming (small T): one workgroup per (expert, 8-column group), weights
//     read once straight into registers -- HBM-bound;
//   * tiled (large T): LDS-staged operand tiles, DMA pipeline -- MFMA-bound.
#include <type_traits>

#include "route_token.hpp"

namespace moe {
namespace {

// ---------------------------------------------------------------------------
// Streaming path (few rows per expert, T <= kGemm1StreamMaxTokens): bound by
// reading the active experts' W13 once from HBM.
//
//   * a workgroup owns one (active expert, 8-column group): the 8 gate rows
//     8c..8c+7 and the 8 matching up rows 2048+8c.. of W13 form one 16-column
//     MFMA tile (lanes r < 8 gate, r >= 8 up), so even a single-token expert
//     spreads over 256 workgroups and SwiGLU is one xor-8 lane exchange;
//   * its 8 waves split K (7 scale blocks each) and issue all their weight
//     loads before the first MFMA; every 16-row tile of the expert's tokens
//     reuses them from registers (more than one tile per expert only on the
//     fallback below, a grid that is not a multiple of 8);
//   * kDirect (T <= 16): the MFMA rows are the T tokens themselves, so the
//     activation loads need no permutation lookup and go out together with
//     the weight loads; results are written to the permuted rows of the
//     expert's tokens.  Otherwise the rows are the expert's permuted rows (the
//     token gather is fused into the A load);
//   * each wave copies its activation scales global -> LDS with
//     global_load_lds_dword; the 8 K-partials are summed in LDS in a fixed
//     order;
//   * an expert of more than 16 rows (hot experts at 17 <= T <= 64) no longer
//     fits one register tile: the loop would reload its rows per item.  The
//     launch then runs the tiled kernel's tiles instead (gemm1_tiled_run, in
//     this kernel's LDS at one workgroup per CU).  Interleaved A/B, GEMM1 us,
//     four hot experts: T = 17 55.3 -> 38.4, 32 68.5 -> 38.9, 48 107.7 ->
//     41.7, 64 173.8 -> 74.2; launches without such experts unchanged.
// ---------------------------------------------------------------------------
constexpr int kGemm1StreamMaxTokens = 64;
constexpr int kGemm1DirectMaxTokens = 16;
constexpr int kS1Waves = 8;
constexpr int kS1Threads = kS1Waves * kWave;
constexpr int kS1KB = kNHBlk / kS1Waves;  // 7 scale blocks per wave
constexpr int kS1Groups = kI / 8;         // 256 column groups per expert
constexpr int kS1CopySplit = 4;           // weight copy parts: K blocks [0, 4) and [4, 7)
constexpr int kS1CopyOps0 = 2 * kS1CopySplit;            // copies per lane, part 0
constexpr int kS1CopyOps1 = 2 * (kS1KB - kS1CopySplit);  // copies per lane, part 1
constexpr int kS1TiledLdsBytes = 81280;  // G1TiledPaths<4, 2>::kLdsBytes (checked where it is defined)

// Operands of one 16-row tile that go out before it is multiplied.
struct S1TileOps {
  v8i a[kS1KB];     // A rows (token rows of hidden_states), this wave's K range
  float s0, s1;     // two of the tile's activation scale entries (lane l: l and 64 + l)
  float sg[kS1KB];  // weight block scales of the item's gate rows (scalar loads) ...
  float su[kS1KB];  // ... and of its up rows; lane r < 8 takes sg, r >= 8 su
  int ptok;         // kDirect: token of the expert's permuted row threadIdx.x (< M)
};

// SwiGLU output of one tile held by each of waves 0-3 (its rows 4q + wave)
// until the next item's loads are out (a store issued before them would
// delay the wait for them).
struct S1Out {
  uint16_t hi, lo;  // the activation as a bf16 pair (split_bf16)
  int row;          // destination act row, -1: none
};

// kDirect: the workgroup routes the T tokens itself (route_small, from the
// routing inputs in `dr`) instead of reading a routing launch's results;
// workgroup 0 also writes them to the workspace for GEMM2 and the caller.
struct DirectRoute {
  const float* logits;
  const uint16_t* bias;
  float rsf;
  int64_t offset;
  RouteOut out;
};
static_assert(kGemm1DirectMaxTokens == kSmallRouteMaxTokens, "the decode path routes in GEMM1");

template <int WM, int WN>
__device__ __forceinline__ void gemm1_tiled_run(char* lds, const uint8_t* __restrict__ hs,
                                                const float* __restrict__ hs_scale, int T,
                                                const uint8_t* __restrict__ w13, const float* __restrict__ w13_scale,
                                                const int32_t* __restrict__ expert_off,
                                                const int32_t* __restrict__ perm_token, const float* __restrict__ perm_w,
                                                uint16_t* __restrict__ act);

template <bool kDirect>
__global__ void __launch_bounds__(kS1Threads)
gemm1_stream_kernel(const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale, int T,
                    const uint8_t* __restrict__ w13, const float* __restrict__ w13_scale,
                    const int32_t* __restrict__ expert_off, const int32_t* __restrict__ perm_token,
                    uint16_t* __restrict__ act, DirectRoute dr) {
  // Per wave: the weights of the item being started (copy j of lane l at
  // 1024 j + 16 l; the only LDS DMA target), the activation scales and the
  // K-partials.  The permutation (<= 8 * 64 rows) is cached whole.
  // One LDS object: with a second __shared__ array the compiler waits for
  // every outstanding LDS DMA before any LDS read.
  constexpr int kWBytes = 2 * kS1KB * 1024;
  constexpr int kSaOff = kS1Waves * kWBytes;
  constexpr int kRedOff = kSaOff + kS1Waves * kS1KB * 16 * 4;
  constexpr int kInvOff = kRedOff + kS1Waves * 4 * kWave * 4;
  constexpr int kPermOff = kInvOff + 16 * 4;
  constexpr int kSrOff = kPermOff + kTopK * kGemm1StreamMaxTokens * 4;  // kDirect: the routing
  constexpr int kLdsBytes = kSrOff + (kDirect ? (int)sizeof(SmallRoute) : 0);
  static_assert(kLdsBytes >= kS1TiledLdsBytes, "the tiled tiles fit this kernel's LDS");
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes];
  float* red = (float*)(lds + kRedOff);
  int* inv = (int*)(lds + kInvOff);                  // kDirect: token -> permuted row, -1 if none
  int* perm_lds = (int*)(lds + kPermOff);
  const int32_t* eoff = expert_off;
  const int32_t* ptok_src = perm_token;
  if constexpr (kDirect) {
    SmallRoute& sr = *(SmallRoute*)(lds + kSrOff);
    route_small(dr.logits, dr.bias, dr.rsf, T, dr.offset, sr, dr.out, blockIdx.x == 0);
    eoff = sr.expert_off;
    ptok_src = sr.perm_token;
  }
  ExpertRows X;
  X.load(eoff);
  if constexpr (!kDirect) {
    // An expert of more than 16 rows: its rows no longer fit one register
    // tile and the streaming loop would reload them per item; run the tiled
    // kernel's tiles instead (in this kernel's LDS, one workgroup per CU).
    if (__ballot(X.cnt > 16) != 0 && gridDim.x % 8 == 0) {
      gemm1_tiled_run<4, 2>(lds, hs, hs_scale, T, w13, w13_scale, expert_off, perm_token, nullptr, act);
      return;
    }
  }
  const uint32_t active = X.active();
  const int items = __popc(active) * kS1Groups;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x & (kWave - 1);
  const int lq = lane >> 4;
  const int lr = lane & 15;
  const int kb0 = wave * kS1KB;
  // scale entries of this wave: entry x = (kb0 + x / 16, row x % 16), x < 112;
  // lane l copies entries l and 64 + l
  const int x1 = kWave + lane;
  char* wbuf = lds + wave * kWBytes;
  float* sa = (float*)(lds + kSaOff) + wave * kS1KB * 16;
  if (!kDirect) {
    const int pairs = X.end(kELocal - 1);
    for (int i = threadIdx.x; i < pairs; i += kS1Threads) perm_lds[i] = perm_token[i];
    lds_barrier();
  }

  // An item's weights of this wave -> its LDS buffer, as 14 wide planes
  // (K block j, rows 8h .. 8h+7 of the item's 16: gate rows 8cg.., then up
  // rows 2048 + 8cg..), 128 bytes per row, chunks swizzled: each copy
  // instruction reads 8 whole 128-byte row segments (the fast lane order for
  // the vector memory path) and the fragment reads are free of bank
  // conflicts.
  // Copied in two parts so that the next item's copy can start before this
  // item's second part has landed: part 0 = K blocks 0-3 (8 copies per lane),
  // part 1 = K blocks 4-6 (6 copies per lane).
  auto copy_w = [&](int item, int part) {
    const int cg = item % kS1Groups;
    const int e = nth_set_bit(active, item / kS1Groups);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      int r, c;
      wide_copy_lane(lane, h, r, c);
      const size_t n = (size_t)e * k2I + (r < 8 ? 8 * cg + r : kI + 8 * cg + (r - 8));
      const uint8_t* src = w13 + n * kH + kb0 * kBlk + 16 * c;
#pragma unroll
      for (int j = 0; j < kS1KB; ++j)
        if ((j < kS1CopySplit) == (part == 0)) dma16_nt(src + j * kBlk, wbuf + (2 * j + h) * 1024);
    }
  };
  // Row tile rt of an item: token of this lane's A row (kDirect: the rows
  // are the tokens themselves), then the tile's row operands -- the same for
  // every item of one expert.
  auto issue_rows = [&](int item, int rt, S1TileOps& o) {
    const int e = nth_set_bit(active, item / kS1Groups);
    const int row0 = X.begin(e) + rt * 16;
    const int rows = kDirect ? T : min(16, X.end(e) - row0);
    const int tok = kDirect ? min(lr, rows - 1) : perm_lds[row0 + min(lr, rows - 1)];
    o.s0 = hs_scale[(size_t)(kb0 + (lane >> 4)) * T + tok];
    o.s1 = x1 < kS1KB * 16 ? hs_scale[(size_t)(kb0 + (x1 >> 4)) * T + tok] : 0.f;
    const uint8_t* ap = hs + (size_t)tok * kH + kb0 * kBlk + 32 * lq;
    if (kDirect) {
      // only the lanes of real rows load (rows >= T are discarded): at
      // T = 1 the other 15 rows' lanes would fetch the same token again
#pragma unroll
      for (int j = 0; j < kS1KB; ++j) o.a[j] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
      if (lr < rows) {
#pragma unroll
        for (int j = 0; j < kS1KB; ++j) o.a[j] = *(const v8i*)(ap + j * kBlk);
      }
    } else {
#pragma unroll
      for (int j = 0; j < kS1KB; ++j) o.a[j] = *(const v8i*)(ap + j * kBlk);
    }
  };
  // kDirect: the expert's permutation entries (LDS), the only per-expert
  // part of the row operands
  auto read_ptok = [&](int item, S1TileOps& o) {
    const int e = nth_set_bit(active, item / kS1Groups);
    o.ptok = 0;
    if ((int)threadIdx.x < X.end(e) - X.begin(e)) o.ptok = ptok_src[X.begin(e) + threadIdx.x];
  };
  // The item's weight block scales: the gate rows and the up rows of an item
  // lie in one 128-row scale block each, so the loads are wave-uniform
  // (scalar loads, counted by lgkmcnt, not vmcnt).  They are issued after
  // the item's weight copies and each lane picks its column's scale only in
  // compute_tile, so no wait for them holds up the copies (small_t64: GEMM1
  // 89 -> 87 us).
  auto issue_sw = [&](int item, S1TileOps& o) {
    const int cg = item % kS1Groups;
    const int e = nth_set_bit(active, item / kS1Groups);
    const float* sg = w13_scale + (((size_t)e * k2I + 8 * cg) / kBlk) * kNHBlk + kb0;
    const float* su = w13_scale + (((size_t)e * k2I + kI + 8 * cg) / kBlk) * kNHBlk + kb0;
#pragma unroll
    for (int j = 0; j < kS1KB; ++j) {
      o.sg[j] = sg[j];
      o.su[j] = su[j];
    }
  };
  // Multiply a landed tile, reduce the 8 K-partials in a fixed order, SwiGLU,
  // store the activation rows.
  auto compute_tile = [&](int item, int rt, const S1TileOps& o, const v8i (&b)[kS1KB], S1Out& out) {
    const int e = nth_set_bit(active, item / kS1Groups);
    const int row0 = X.begin(e);
    const int M = X.end(e) - row0;
    const int rows = kDirect ? T : min(16, M - rt * 16);
    sa[lane] = o.s0;
    if (x1 < kS1KB * 16) sa[x1] = o.s1;
    if (kDirect) {
      if (threadIdx.x < 16) inv[threadIdx.x] = -1;
      lds_barrier();
      if ((int)threadIdx.x < M) inv[o.ptok] = row0 + threadIdx.x;  // read after the barrier below
    }
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < kS1KB; ++j) {
      const v4f p = mfma_f8_16x16x128(o.a[j], b[j]);
      const v4f sc = *(const v4f*)&sa[j * 16 + 4 * lq];
      const float sw = lr < 8 ? o.sg[j] : o.su[j];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(p[i], sc[i] * sw, acc[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(wave * 4 + i) * kWave + lane] = acc[i];
    lds_barrier();
    if (wave < 4) {
      // wave i sums the partials of output rows 4q + i in wave order
      const int i = wave;
      float v = red[i * kWave + lane];
#pragma unroll
      for (int w = 1; w < kS1Waves; ++w) v += red[(w * 4 + i) * kWave + lane];
      // SwiGLU (moe.py:190-193): lanes r < 8 hold gate, lanes r + 8 the up column
      const float x2 = __shfl_xor(v, 8, kWave);
      const int r = 4 * lq + i;
      const int prow = kDirect ? (r < rows ? inv[r] : -1) : (r < rows ? row0 + rt * 16 + r : -1);
      split_bf16(silu_mul(x2, v), out.hi, out.lo);
      out.row = lr < 8 ? prow : -1;
    }
    lds_barrier();  // red / sa / inv consumed before they are rewritten
  };
  auto store_out = [&](int item, const S1Out& out) {
    if (wave < 4 && out.row >= 0) {
      uint16_t* p = act + (size_t)out.row * kActRowElems + act_col(8 * (item % kS1Groups) + lr);
      p[0] = out.hi;
      p[64] = out.lo;
    }
  };

  // Persistent: the grid is at most what fits on the device at once, and
  // each workgroup takes a contiguous range of the (active expert, column
  // group) items, so no workgroup is launched for an expert without rows and
  // consecutive items of a workgroup mostly share their expert, whose row
  // operands then stay in registers.  Each item starts by waiting for its
  // weights and operands (issued during the previous item), moves the
  // weights LDS -> registers, and at once sends out the next item's weight
  // copy and loads, which stream while this item is multiplied, reduced and
  // stored.
  const int per = (items + (int)gridDim.x - 1) / (int)gridDim.x;
  const int i0 = blockIdx.x * per;
  const int i1 = min(items, i0 + per);
  // One set of operands.  The weight scales of the next item are scalar
  // loads into `nsw` while an item runs.  The row operands change only with
  // the expert (kDirect: never -- the rows are the T tokens for every
  // expert, only the permutation entries change) and are then reloaded
  // after the item's tiles, and waited for at once: once per expert change
  // (or per item, for an expert of more than 16 rows, whose later row tiles
  // pass through the same registers).  A second set filled while the item
  // runs and copied over at its end made the compiler wait at every item
  // for every load, the next item's whole weight copy included, since it
  // could not tell the copied registers had landed.
  S1TileOps cur;
  S1Out pend;       // the previous tile's outputs, stored once the next loads are out
  if (i0 < i1) {
    issue_rows(i0, 0, cur);
    if (kDirect) read_ptok(i0, cur);
    copy_w(i0, 0);
    copy_w(i0, 1);
    issue_sw(i0, cur);
    // kDirect: the token rows land while the copies are issued.  Left
    // pending into the item loop (which loads no register of its own), they
    // made the compiler wait for every outstanding load before the loop,
    // the first item's whole weight copy included.
    if (kDirect) wait_vmcnt<kS1CopyOps0 + kS1CopyOps1>();
  }
  // fragment of block j: lane (q, r) holds row r, K bytes 32q .. 32q+31
  const int slot_lo = wide_slot(lr, 2 * lq), slot_hi = wide_slot(lr, 2 * lq + 1);
  auto read_b = [&](v8i (&b)[kS1KB], int j) {
    const v4i lo = *(const v4i*)(wbuf + 2 * j * 1024 + slot_lo);
    const v4i hi = *(const v4i*)(wbuf + 2 * j * 1024 + slot_hi);
    b[j] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };
  // Vector-memory order per item: [copy part 0] ... [copy part 1] [the
  // previous tile's store], then on an expert change the next row operands,
  // waited for at once.  The weight scales are scalar loads (lgkmcnt), so
  // only copies and at most one store are counted by the waits below.
#pragma unroll 1
  for (int item = i0; item < i1; ++item) {
    const bool more = item + 1 < i1;
    const bool new_rows = more && (item + 1) / kS1Groups != item / kS1Groups;
    // Part 0 has landed, and the row operands issued before it; part 1 and
    // the store after it may still be in flight.
    wait_vmcnt_lgkm0<kS1CopyOps1>();
    asm volatile("" ::: "memory");
    v8i b[kS1KB];
#pragma unroll
    for (int j = 0; j < kS1CopySplit; ++j) read_b(b, j);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // part 0 is read: free for the next item's
    S1TileOps nsw;  // the next item's weight scales (only sg, su are used)
    if (more) {
      copy_w(item + 1, 0);
      issue_sw(item + 1, nsw);
    }
    // Part 1 has landed; the next item's part 0 may still be in flight.
    if (more)
      wait_vmcnt_lgkm0<kS1CopyOps0>();
    else
      wait_vmcnt_lgkm0<0>();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int j = kS1CopySplit; j < kS1KB; ++j) read_b(b, j);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // part 1 is read
    if (more) copy_w(item + 1, 1);
    if (item != i0) store_out(item - 1, pend);
    compute_tile(item, 0, cur, b, pend);
    if (kDirect) {
      if (new_rows) read_ptok(item + 1, cur);
    } else {
      const int e = nth_set_bit(active, item / kS1Groups);
      const bool multi_tile = X.end(e) - X.begin(e) > 16;
#pragma unroll 1
      for (int rt = 1; rt * 16 < X.end(e) - X.begin(e); ++rt) {
        issue_rows(item, rt, cur);
        wait_vmcnt_lgkm0<0>();  // also the next item's copy: experts of > 16 rows are rare here
        asm volatile("" ::: "memory");
        store_out(item, pend);
        compute_tile(item, rt, cur, b, pend);
      }
      if (more && (new_rows || multi_tile)) {
        issue_rows(item + 1, 0, cur);
        wait_vmcnt_lgkm0<0>();
        asm volatile("" ::: "memory");
      }
    }
    if (more) {
#pragma unroll
      for (int j = 0; j < kS1KB; ++j) {
        cur.sg[j] = nsw.sg[j];
        cur.su[j] = nsw.su[j];
      }
    }
  }
  if (i0 < i1) store_out(i1 - 1, pend);
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
//     staging) into a ring of kStages LDS buffers, the loads of stage
//     kb + kStages - 1 in flight while stage kb is multiplied;
//   * LDS holds each 16-row x 128-K operand fragment as two wide 1 KB planes
//     (8 rows x 128 B, row-major, chunks swizzled): every copy instruction
//     reads 8 whole 128-byte row segments and the MFMA operand reads are free
//     of bank conflicts;
//   * per K block: P = A_f8 * B_f8 (v_mfma_f32_16x16x128_f8f6f4, exact
//     products), acc += P * (a_scale[row] * w_scale[n/128]).
// ---------------------------------------------------------------------------
// Kernel choice by T: the tiled kernel up to kGemm1TiledLargeMinTokens - 1,
// both launched up to kGemm1BothMaxTokens (each exits unless the row counts
// choose it, wide_tiles_full), the wide 256 x 256 tiles beyond.  Both give
// the same output bits.  The wide tiles pay when a few experts hold most rows
// (their 256-row tiles then mostly full); with rows spread over many experts
// the tiled kernel's 64- and 128-row tiles copy less and fill two workgroups
// per CU.  Interleaved A/B, GEMM1 us, wide -> tiled: prefill routing
// T = 1025 184.0 -> 139.5, 1280 188.9 -> 146.6, 1536 179.4 -> 167.3, 2048
// 198.8 -> 198.1; small_t64 routing T = 1100 182.8 -> 147.0, 1536 188.3 ->
// 166.8, 2048 193.5 -> 191.5; four hot experts T = 1025 196.7 -> 216.6, 1536
// 268.1 -> 297.2, 2048 317.7 -> 369.0 (wide tile fill 0.20-0.39 without hot
// experts, 0.54-0.74 with them).  Past T = 1536 the spread case is a tie,
// and launching both would cost the exiting kernel's ~3 us.
constexpr int kGemm1TiledLargeMinTokens = 1025;
constexpr int kGemm1BothMaxTokens = 1536;

// True when the wide kernel's 256-row tiles would be at least 45 % full.
// Wave-level; the same in every workgroup of both kernels.
__device__ __forceinline__ bool wide_tiles_full(const ExpertRows& X) {
  const int rows = __builtin_amdgcn_readlane(lane_scan_incl(X.cnt), kWave - 1);
  return 100 * rows >= 45 * 256 * X.count_tiles(256);
}

template <int WM, int WN, int MI, int ST>
struct G1Tiled {
  static constexpr int kWN = WN;
  static constexpr int kMI = MI;
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
  // Activation scales: every lane of every wave DMAs one dword (a branch on
  // the lane would split the main loop into basic blocks and keep the MFMA
  // results live across them), so each wave owns a 64-dword slot whose first
  // kScaleRowsPerWave entries are its rows' scales.
  static constexpr int kStageBytes = kSOff + kWaves * kWave * 4;
  static constexpr int kWscBytes = WN * 2 * kNHBlk * 4;  // weight block scales (after the stages)
  static constexpr int kStages = ST;
  static_assert(kStages >= 2 && kStages <= 6, "pipeline depth (wait_stages_ahead)");
  static constexpr int kRingBytes = kStages * kStageBytes;
  static constexpr int kPlanes = 2 * (kAFrags + kBFrags);
  static_assert(kPlanes % kWaves == 0, "planes must split evenly over waves");
  static constexpr int kPlanesPerWave = kPlanes / kWaves;
  static constexpr int kScaleRowsPerWave = BM / kWaves;
  static_assert(kScaleRowsPerWave % 4 == 0 && kScaleRowsPerWave <= kWave, "scale rows per wave");
  static constexpr int kDmaPerStage = kPlanesPerWave + 1;
};

// Two tile heights.  Short tiles hold up to 64 rows of one expert (one 16-row
// block per wave, a 3-stage ring); tall tiles 65-128 rows (two blocks per
// wave, a 2-stage ring), so the W13 columns of those rows are copied (and,
// for an expert of up to 128 rows, read from HBM) once instead of once per 64
// rows.  The kernel waits on that weight stream: with every tile's W13
// L2-resident (a timing-only copy) it ran 26 % faster at T = 1024, while more
// lookahead through L2 prefetches made it slower.  Rows past a
// tile's last row copy its last row again, which costs the copy path nothing
// (lanes given an out-of-range buffer offset instead changed no time).  Both
// rings fit one LDS array of the short ring's size: two workgroups per CU.
// A tall tile costs about 1.5 short ones; with few tiles per workgroup one
// tall tile can outlast two short ones, so each launch chooses between tall
// tiles and short tiles only from the row counts (G1TiledPaths::use_tall).
template <int WM, int WN>
struct G1TiledPaths {
  using Short = G1Tiled<WM, WN, 1, 3>;
  using Tall = G1Tiled<WM, WN, 2, 2>;
  static_assert(2 * Short::BM == Tall::BM && Short::kNT == Tall::kNT, "a tall tile is two short ones");
  static constexpr int BM = Tall::BM;           // tile height of the tile map
  static constexpr int kNT = Short::kNT;
  static constexpr int kThreads = Short::kThreads;
  static constexpr int kGroupM = 4;             // at most this many row tiles (of one expert) per L2 group
  static constexpr int kRingBytes = Short::kRingBytes > Tall::kRingBytes ? Short::kRingBytes : Tall::kRingBytes;
  static constexpr int kRowWBytes = Tall::BM * 4;  // the tile's routing weights (every_token_experts)
  static constexpr int kLdsBytes = kRingBytes + Short::kWscBytes + kRowWBytes;
  static_assert(WM != 4 || WN != 2 || kLdsBytes <= kS1TiledLdsBytes, "the streaming kernel's LDS check");
  // Tall tiles (and the tall-first map) or short tiles only, for a grid of
  // `slots` resident workgroups.  In short-tile units a tall tile costs 1.5,
  // so the work is W = 1.5 tall + short against S short tiles.  Tall tiles
  // pay (a) when they fit the work into one round of slots that the short
  // tiles overflow, or (b) when the short tiles take at least 1.6 rounds and W
  // saves 5 %.  Below one round the short map runs an expert's two short
  // tiles side by side, faster than one tall tile; between one and 1.6 rounds
  // both maps end in a partial round, and tall tiles lengthen the first.
  // Interleaved A/B, GEMM1 us (short tiles only -> this rule's choice):
  // prefill routing T = 1024 157.7 -> 138.6, 896 154.9 -> 136.3, 768 142.6 ->
  // 129.1, 640 137.6 -> 126.6; hot experts T = 1024 269.2 -> 214.6, 512
  // 168.6 -> 149.3, 256 118.7 -> 104.8, 128 94.5 -> 82.7.  Tall tiles where
  // the rule keeps the short map: prefill T = 512 106.4 -> 111.8, 384 103.5 ->
  // 109.8; hot experts T = 192 93.8 -> 99.9, 96 65.1 -> 76.1, 65 62.1 -> 71.9.
  __device__ static bool use_tall(const ExpertRows& X, int slots) {
    int n_tall, n_short;
    tall_short_row_tiles(X, BM, n_tall, n_short);
    const int s_rows = X.count_tiles(Short::BM);  // short-map row tiles
    const int w2 = 3 * n_tall + 2 * n_short;       // 2 W in row tiles
    const bool one_round = s_rows * kNT > slots && w2 * kNT <= 2 * slots;
    const bool saves = 5 * s_rows * kNT >= 8 * slots && 10 * w2 <= 19 * s_rows;
    return n_tall > 0 && (one_round || saves);
  }
};

// One tile: `rows` rows of expert e from permuted row row0, gate columns
// j0 .. j0 + kGateCols - 1 and the matching up columns.  `lds` is the
// kernel's one LDS object (the stage ring), `wsc` the weight scale table
// after it.  Every wave of the workgroup calls it; the caller's barrier
// separates consecutive tiles.
template <class C>
__device__ __forceinline__ void gemm1_tile(char* lds, float* wsc, const uint8_t* __restrict__ hs,
                                           const float* __restrict__ hs_scale, int T,
                                           const uint8_t* __restrict__ w13, const float* __restrict__ w13_scale,
                                           const int32_t* __restrict__ perm_token, uint16_t* __restrict__ act,
                                           int e, int row0, int rows, int j0, bool w_once,
                                           const float* __restrict__ perm_w, bool fold_w) {
  constexpr int WN = C::kWN, MI = C::kMI;
  // The thread index is opaque to the optimiser: values derived from it are
  // computed per tile, not hoisted out of the tile loop and kept live
  // (spilled) across the tall path, which needs all 128 VGPRs.
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform (SGPR)
  const int lane = tid & (kWave - 1);
  const int lq = lane >> 4;
  const int lr = lane & 15;
  const int wm = wave / WN;
  const int wn = wave % WN;

  // ---- DMA planes of this wave: planes wave + 8k; the first kAPlanes are
  // hidden rows (A), the rest W13 rows (B).  Sources are a wave-uniform base
  // plus a 32-bit lane offset, one VGPR per plane (T <= 1024 here, so every
  // offset fits).
  constexpr int kAPlanes = 2 * C::kAFrags / C::kWaves;
  static_assert((2 * C::kAFrags) % C::kWaves == 0, "A planes split evenly over the waves");
  const uint8_t* w13e = w13 + (size_t)e * k2I * kH;
  uint32_t off[C::kPlanesPerWave];
  int dst[C::kPlanesPerWave];
#pragma unroll
  for (int k = 0; k < C::kPlanesPerWave; ++k) {
    const int plane = wave + k * C::kWaves;
    const int frag = plane >> 1, half = plane & 1;
    int fr, chunk;
    wide_copy_lane(lane, half, fr, chunk);
    if (k < kAPlanes) {
      const int r = min(frag * 16 + fr, rows - 1);
      off[k] = (uint32_t)perm_token[row0 + r] * kH + 16 * chunk;
      dst[k] = frag * C::kFrag + half * 1024;
    } else {
      const int bf = frag - C::kAFrags;
      const int n = bf < 2 * WN ? j0 + 16 * bf + fr : kI + j0 + 16 * (bf - 2 * WN) + fr;
      off[k] = (uint32_t)n * kH + 16 * chunk;
      dst[k] = C::kBOff + bf * C::kFrag + half * 1024;
    }
  }
  // lanes past the wave's rows copy the first row's scale again (one cache
  // line instead of one per lane; their slot entries are never read)
  const int srow = wave * C::kScaleRowsPerWave + (lane < C::kScaleRowsPerWave ? lane : 0);
  const uint32_t stok = (uint32_t)perm_token[row0 + min(srow, rows - 1)];
  const int sdst = C::kSOff + wave * kWave * 4;

  // The W13 tile of an expert with a single row tile is read exactly once:
  // its copies take the nontemporal policy (T = 128: GEMM1 88.1 -> 77.5 us,
  // T = 1024 181.3 -> 174.4 us).  Experts of several row tiles re-read it
  // through L2 and keep the default (nt everywhere made T = 1024 8 % slower).
  auto issue = [&](int kb) {
    char* base = lds + (kb % C::kStages) * C::kStageBytes;
#pragma unroll
    for (int k = 0; k < C::kPlanesPerWave; ++k) {
      if (k < kAPlanes)
        dma16(hs + kb * kBlk + off[k], base + dst[k]);
      else if (w_once)
        dma16_nt(w13e + kb * kBlk + off[k], base + dst[k]);
      else
        dma16(w13e + kb * kBlk + off[k], base + dst[k]);
    }
    dma4(hs_scale + (size_t)kb * T + stok, base + sdst);
  };

  // Weight block scales of every wave's gate / up columns, staged in LDS once
  // (no scalar loads in the main loop: they would force full lgkmcnt waits).
  for (int i = tid; i < WN * 2 * kNHBlk; i += C::kThreads) {  // [WN][2][56]
    const int w_n = i / (2 * kNHBlk), up = (i / kNHBlk) & 1, kb = i % kNHBlk;
    const int blk = (up ? kI : 0) + j0 + 32 * w_n;
    wsc[i] = w13_scale[((size_t)e * kN2IBlk + blk / kBlk) * kNHBlk + kb];
  }
  // the rows' routing weights, for the epilogue (every_token_experts)
  float* roww = wsc + WN * 2 * kNHBlk;
  if (fold_w)
    for (int i = tid; i < rows; i += C::kThreads) roww[i] = perm_w[row0 + i];

  v4f acc[MI][4];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) acc[mi][nj] = v4f{0.f, 0.f, 0.f, 0.f};

  // Pipeline: the DMA of a stage is issued kStages - 1 steps before its
  // operands are read, and the kernel is capped at 128 VGPRs (launch bounds
  // of 4 waves per SIMD) so that two workgroups share a CU; the LDS reads of
  // one workgroup overlap the MFMAs of the other.
  struct Frags {
    v8i a[MI], b[4];
    v4f sa[MI];
    float sg, su;
  };
  const int slot_lo = wide_slot(lr, 2 * lq), slot_hi = wide_slot(lr, 2 * lq + 1);
  auto frag = [&](int s, int off) {
    const char* f = lds + (s % C::kStages) * C::kStageBytes + off;
    const v4i lo = *(const v4i*)(f + slot_lo), hi = *(const v4i*)(f + slot_hi);
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };
  auto read_b = [&](int s, Frags& F) {
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) F.b[nj] = frag(s, C::kBOff + (nj < 2 ? 2 * wn + nj : 2 * WN + 2 * wn + (nj - 2)) * C::kFrag);
    F.sg = wsc[(2 * wn) * kNHBlk + s];
    F.su = wsc[(2 * wn + 1) * kNHBlk + s];
  };
  auto read_a = [&](int s, int mi, Frags& F) {
    F.a[mi] = frag(s, (wm * MI + mi) * C::kFrag);
    const int r = wm * 16 * MI + 16 * mi + 4 * lq;  // 4 rows in one wave's slot
    const int slot = (r / C::kScaleRowsPerWave) * kWave + r % C::kScaleRowsPerWave;
    F.sa[mi] = *(const v4f*)(lds + (s % C::kStages) * C::kStageBytes + C::kSOff + slot * 4);
  };
  auto compute_row = [&](const Frags& F, int mi) {
    v4f sgm, sum;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sgm[i] = F.sa[mi][i] * F.sg;
      sum[i] = F.sa[mi][i] * F.su;
    }
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) {
      const v4f p = mfma_f8_16x16x128(F.a[mi], F.b[nj]);
      const v4f sc = nj < 2 ? sgm : sum;
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[mi][nj][i] = __builtin_fmaf(p[i], sc[i], acc[mi][nj][i]);
    }
  };
  auto compute = [&](const Frags& F) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) compute_row(F, mi);
  };

  // One fragment set, read at the start of each step: with four waves per
  // SIMD the other waves cover the LDS latency.  Step kb: stage kb has
  // landed (later stages may stay in flight) and, after the barrier, every
  // wave is done with stage kb - 1, whose buffer takes stage kb + kStages - 1.
  Frags f;
#pragma unroll
  for (int s = 0; s < C::kStages - 1; ++s) issue(s);
#pragma unroll 1
  for (int kb = 0; kb < kNHBlk; ++kb) {
    wait_stages_ahead<C::kDmaPerStage>(min(C::kStages - 2, kNHBlk - 1 - kb));
    block_barrier();
    if (kb + C::kStages - 1 < kNHBlk) issue(kb + C::kStages - 1);
    read_b(kb, f);
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) read_a(kb, mi, f);
    compute(f);
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
          float v = silu_mul(x2, x1);
          if (fold_w) v = v * roww[r];  // every_token_experts: the routing weight
          uint16_t hi, lo;
          split_bf16(v, hi, lo);
          uint16_t* p = act + (size_t)(row0 + r) * kActRowElems + act_col(j0 + 32 * wn + 16 * nj + lr);
          p[0] = hi;
          p[64] = lo;
        }
      }
}

// The tiled kernel's tile loop, over the whole grid; also run by the
// streaming kernel when an expert has more than 16 rows.  `lds` holds at
// least G1TiledPaths::kLdsBytes; the grid must be a multiple of 8.
template <int WM, int WN>
__device__ __forceinline__ void gemm1_tiled_run(char* lds, const uint8_t* __restrict__ hs,
                                                const float* __restrict__ hs_scale, int T,
                                                const uint8_t* __restrict__ w13, const float* __restrict__ w13_scale,
                                                const int32_t* __restrict__ expert_off,
                                                const int32_t* __restrict__ perm_token, const float* __restrict__ perm_w,
                                                uint16_t* __restrict__ act) {
  using P = G1TiledPaths<WM, WN>;
  float* wsc = (float*)(lds + P::kRingBytes);  // [WN][2][56]

  // Persistent: the grid is at most what fits on the device at once; each
  // workgroup walks its tiles (no workgroup is launched past the last tile).
  // Short map: contiguous eighths of the 64-row tile order per XCD.  Tall
  // map: xcd_tall_first_tile, block b taking XCD b % 8's tiles b / 8 in the
  // first round, then in reverse order (snake), so that the blocks that ran a
  // tall tile first take a second tile last.  The expert offsets are read
  // again for every tile (one L2 load) rather than kept in two VGPRs across
  // the tall path, which needs all 128.
  bool tall_map;
  {
    ExpertRows X;
    X.load(expert_off);
    tall_map = P::use_tall(X, gridDim.x);    // the same in every workgroup
  }
  const int xcd = blockIdx.x % 8, cap = gridDim.x / 8, slot = blockIdx.x / 8;
#pragma unroll 1
  for (int it = 0;; ++it) {
    ExpertRows X;
    X.load(expert_off);
    int mt, nt, e, row0, rows;
    if (tall_map) {
      const int li = (it & 1) ? (it + 1) * cap - 1 - slot : it * cap + slot;
      if (!xcd_tall_first_tile(X, xcd, li, P::BM, P::kNT, P::kGroupM, mt, nt)) break;
      X.find_tile(mt, P::BM, e, row0, rows);
    } else {
      const int t = xcd_tile_nth(blockIdx.x, gridDim.x, X.count_tiles(P::Short::BM) * P::kNT, it);
      if (t < 0) break;
      grouped_tile(X, t, P::Short::BM, P::kNT, P::kGroupM, mt, nt);
      X.find_tile(mt, P::Short::BM, e, row0, rows);
    }
    if (it > 0) block_barrier();  // every wave is done with the previous tile's LDS
    const int j0 = nt * P::Short::kGateCols;
    const bool w_once = X.end(e) - X.begin(e) <= (tall_map ? P::BM : P::Short::BM);  // one row tile
    const bool fold_w = (every_token_experts(X, T) >> e) & 1u;
    if (rows > P::Short::BM)  // workgroup-uniform
      gemm1_tile<typename P::Tall>(lds, wsc, hs, hs_scale, T, w13, w13_scale, perm_token, act, e, row0, rows, j0,
                                   w_once, perm_w, fold_w);
    else
      gemm1_tile<typename P::Short>(lds, wsc, hs, hs_scale, T, w13, w13_scale, perm_token, act, e, row0, rows, j0,
                                    w_once, perm_w, fold_w);
  }
}


// both: launched together with the wide kernel; runs only if the row counts
// choose the tiled tiles (!wide_tiles_full).
template <int WM, int WN>
__global__ void __launch_bounds__(64 * WM * WN, 4)
gemm1_tiled_kernel(const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale, int T,
                   const uint8_t* __restrict__ w13, const float* __restrict__ w13_scale,
                   const int32_t* __restrict__ expert_off, const int32_t* __restrict__ perm_token,
                   const float* __restrict__ perm_w, uint16_t* __restrict__ act, int both) {
  using P = G1TiledPaths<WM, WN>;
  // One LDS object: the stage ring, then the weight scale table.  (A second
  // __shared__ array makes the compiler wait for every outstanding LDS DMA
  // before any LDS read, which would serialise the pipeline.)
  __shared__ __attribute__((aligned(1024))) char lds[P::kLdsBytes];
  float* wsc = (float*)(lds + P::kRingBytes);  // [WN][2][56]
  {
    ExpertRows X;
    X.load(expert_off);
    if (both && wide_tiles_full(X)) return;  // the wide kernel takes this launch
  }
  gemm1_tiled_run<WM, WN>(lds, hs, hs_scale, T, w13, w13_scale, expert_off, perm_token, perm_w, act);
}

template <int WM, int WN>
hipError_t launch_gemm1_tiled(const uint8_t* hs, const float* hs_scale, int T, const uint8_t* w13,
                              const float* w13_scale, const Layout& L, char* ws, hipStream_t stream, int both) {
  using P = G1TiledPaths<WM, WN>;
  const int64_t pairs = (int64_t)T * kTopK;
  const int64_t mtiles = (pairs + P::Short::BM - 1) / P::Short::BM + (pairs < kELocal ? pairs : kELocal);
  static ResidentGrid resident(gemm1_tiled_kernel<WM, WN>, P::kThreads);
  const int64_t upper = ((mtiles * P::kNT + 7) / 8) * 8;
  const int resident_n = resident.count();
  const int64_t cap = resident_n >= 8 ? resident_n / 8 * 8 : 8;
  const int64_t blocks = upper < cap ? upper : cap;
  hipLaunchKernelGGL((gemm1_tiled_kernel<WM, WN>), dim3((unsigned)blocks), dim3(P::kThreads), 0,
                     stream, hs, hs_scale, T, w13, w13_scale, (const int32_t*)(ws + L.expert_off),
                     (const int32_t*)(ws + L.perm_token), (const float*)(ws + L.perm_w), (uint16_t*)(ws + L.act),
                     both);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Wide path (large T): 256 rows x 256 MFMA columns per workgroup.
//
// A 256 x 256 tile moves (256 + 256) x 128 B per K block for 2 x 256 x 256 x
// 128 FLOP, a third less per FLOP than 256 x 128 tiles, which were slower.
// What bounds it is the stage itself (barrier, operand reads, copy issue):
// with every operand L2-resident (a timing-only copy) it ran only 2 % faster.
//
//   * 8 waves as 4 (rows) x 2 (columns); wave tile = 64 rows x (64 gate + the
//     64 matching up columns), 4 x 8 MFMA blocks, 128 accumulator VGPRs;
//   * the workgroup's 128 gate columns (and its 128 up columns) are one
//     128-column weight scale block, so one gate and one up scale per K block;
//   * two LDS stages of 66 KB: the copy of K block kb + 1 runs while K block
//     kb is multiplied, its DMAs issued between the first MFMAs;
//   * the DMA sources are a wave-uniform base plus a 32-bit lane offset
//     (saddr form), one VGPR per copied plane.
// ---------------------------------------------------------------------------
struct G1Wide {
  static constexpr int kWaves = 8;
  static constexpr int kThreads = kWave * kWaves;
  static constexpr int WM = 4, WN = 2;
  static constexpr int MI = 4;                   // 16-row blocks per wave
  static constexpr int NJ = 4;                   // 16-column gate blocks per wave (and as many up)
  static constexpr int BM = 16 * MI * WM;        // 256 rows
  static constexpr int kGateCols = 16 * NJ * WN; // 128 act columns
  static constexpr int kNT = kI / kGateCols;     // 16 column tiles
  static constexpr int kAFrags = BM / 16;        // 16
  static constexpr int kBFrags = 2 * kGateCols / 16;  // 16: 8 gate + 8 up
  static constexpr int kFrag = 2048;
  static constexpr int kBOff = kAFrags * kFrag;
  static constexpr int kSOff = kBOff + kBFrags * kFrag;
  static constexpr int kStageBytes = kSOff + kWaves * kWave * 4;  // + one 64-dword scale slot per wave
  static constexpr int kStages = 2;
  static constexpr int kWscBytes = 2 * kNHBlk * 4;
  static constexpr int kPlanes = 2 * (kAFrags + kBFrags);
  static constexpr int kPlanesPerWave = kPlanes / kWaves;       // 8: 4 A + 4 B
  static constexpr int kScaleRowsPerWave = BM / kWaves;         // 32
  static constexpr int kGroupM = 4;
  static_assert(kGateCols == kBlk, "one weight scale block per tile");
  static_assert(kPlanes % kWaves == 0 && (kAFrags * 2) % kWaves == 0, "planes split evenly");
  static_assert(kScaleRowsPerWave % 4 == 0 && kScaleRowsPerWave <= kWave, "scale rows per wave");
  static_assert(kStages * kStageBytes + kWscBytes <= 160 * 1024, "LDS");
};

// both: launched together with the tiled kernel; runs only if the row counts
// choose the wide tiles (wide_tiles_full).
__global__ void __launch_bounds__(G1Wide::kThreads)
gemm1_wide_kernel(const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale, int T,
                  const uint8_t* __restrict__ w13, const float* __restrict__ w13_scale,
                  const int32_t* __restrict__ expert_off, const int32_t* __restrict__ perm_token,
                  const float* __restrict__ perm_w, uint16_t* __restrict__ act, int both) {
  using C = G1Wide;
  __shared__ __attribute__((aligned(1024))) char lds[C::kStages * C::kStageBytes + C::kWscBytes];

  ExpertRows X;
  X.load(expert_off);
  if (both && !wide_tiles_full(X)) return;  // the tiled kernel takes this launch
  const uint32_t fused = every_token_experts(X, T);
  // An eighth of every expert's tiles per XCD (xcd_expert_tile): block b
  // takes tiles b / 8, b / 8 + cap, ... of XCD b % 8, cap being the blocks per
  // XCD.  The grid has a block per possible tile, so a block nearly always
  // takes one tile; the loop covers an XCD that holds more than cap (an XCD
  // holds up to 32 tiles more than an eighth of all).
  const int xcd = blockIdx.x % 8, cap = gridDim.x / 8;
#pragma unroll 1
  for (int li = blockIdx.x / 8;; li += cap) {
  int mt, nt;
  if (!xcd_expert_tile(X, xcd, li, C::BM, C::kNT, C::kGroupM, mt, nt)) break;
  if (li >= cap) block_barrier();  // every wave is done with the previous tile's LDS
  int e, row0, rows;
  X.find_tile(mt, C::BM, e, row0, rows);
  const int j0 = nt * C::kGateCols;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x & (kWave - 1);
  const int lq = lane >> 4;
  const int lr = lane & 15;
  const int wm = wave / C::WN;
  const int wn = wave % C::WN;
  const int slot_lo = wide_slot(lr, 2 * lq), slot_hi = wide_slot(lr, 2 * lq + 1);

  // ---- DMA planes of this wave: planes wave + 8k; k < 4 are A, k >= 4 are B
  const uint8_t* w13e = w13 + (size_t)e * k2I * kH;
  uint32_t off[C::kPlanesPerWave];
  int dst[C::kPlanesPerWave];
#pragma unroll
  for (int k = 0; k < C::kPlanesPerWave; ++k) {
    const int plane = wave + k * C::kWaves;
    const int frag = plane >> 1, half = plane & 1;
    int fr, chunk;
    wide_copy_lane(lane, half, fr, chunk);
    if (frag < C::kAFrags) {
      const int r = min(frag * 16 + fr, rows - 1);
      off[k] = (uint32_t)perm_token[row0 + r] * kH + 16 * chunk;
      dst[k] = frag * C::kFrag + half * 1024;
    } else {
      const int bf = frag - C::kAFrags;  // 0..7 gate, 8..15 up
      const int n = bf < 8 ? j0 + 16 * bf + fr : kI + j0 + 16 * (bf - 8) + fr;
      off[k] = (uint32_t)n * kH + 16 * chunk;
      dst[k] = C::kBOff + bf * C::kFrag + half * 1024;
    }
  }
  // lanes past the wave's rows copy the first row's scale again (their slot
  // entries are never read)
  const uint32_t stok =
      (uint32_t)perm_token[row0 + min(wave * C::kScaleRowsPerWave + (lane < C::kScaleRowsPerWave ? lane : 0), rows - 1)];
  const int sdst = C::kSOff + wave * kWave * 4;

  auto issue_plane = [&](int kb, int k, auto nt_c) {
    char* base = lds + (kb & 1) * C::kStageBytes;
    const bool a_plane = k < C::kPlanesPerWave / 2;
    if (a_plane) {
      // A fragments wholly past the tile's rows are never read: no copy
      if (((wave + k * C::kWaves) >> 1) * 16 < rows) dma16(hs + kb * kBlk + off[k], base + dst[k]);
    } else if constexpr (decltype(nt_c)::value) {
      dma16_nt(w13e + kb * kBlk + off[k], base + dst[k]);
    } else {
      dma16(w13e + kb * kBlk + off[k], base + dst[k]);
    }
  };
  auto issue_scale = [&](int kb) {
    dma4(hs_scale + (size_t)kb * T + stok, lds + (kb & 1) * C::kStageBytes + sdst);
  };
  auto issue = [&](int kb, auto nt_c) {
#pragma unroll
    for (int k = 0; k < C::kPlanesPerWave; ++k) issue_plane(kb, k, nt_c);
    issue_scale(kb);
  };

  // weight block scales of the tile's gate block and up block, per K block
  float* wsc = (float*)(lds + C::kStages * C::kStageBytes);  // [2][56]
  for (int i = threadIdx.x; i < 2 * kNHBlk; i += C::kThreads) {
    const int up = i / kNHBlk, kb = i % kNHBlk;
    wsc[i] = w13_scale[((size_t)e * kN2IBlk + (up ? kI : 0) / kBlk + j0 / kBlk) * kNHBlk + kb];
  }

  v4f acc[C::MI][2 * C::NJ];
#pragma unroll
  for (int mi = 0; mi < C::MI; ++mi)
#pragma unroll
    for (int nj = 0; nj < 2 * C::NJ; ++nj) acc[mi][nj] = v4f{0.f, 0.f, 0.f, 0.f};

  // Multiply stage kb; with kc >= 0 also copy stage kc, its DMAs spread over
  // the first column blocks (two planes behind each block's first MFMAs):
  // issued as one burst after the barrier, they filled the memory pipeline
  // and every wave stalled in the issue before its first MFMA (T = 8192:
  // 1,198 -> 1,103 us; one plane per block needed more registers than fit).
  auto compute = [&](int kb, int kc, auto nt_c) {
    const char* sb = lds + (kb & 1) * C::kStageBytes;
    auto frag = [&](int off_) {
      const char* f = sb + off_;
      const v4i lo = *(const v4i*)(f + slot_lo), hi = *(const v4i*)(f + slot_hi);
      return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    // column block nj: gate blocks 0 .. NJ-1, then the matching up blocks
    auto bfrag = [&](int nj) {
      return frag(C::kBOff + (nj < C::NJ ? C::NJ * wn + nj : 8 + C::NJ * wn + nj - C::NJ) * C::kFrag);
    };
    // Operands swapped (W13 rows as the MFMA's A): lane (q, r) receives row
    // r, columns 4q .. 4q+3 of each block, so one row scale per lane and row
    // block, and the epilogue stores 4 adjacent columns at once.  LDS reads
    // in order of first use: block 0's B fragment and the A fragments, then,
    // behind block 0's MFMAs, the scales (first needed one block later).
    v8i bn = bfrag(0);
    v8i a[C::MI];
#pragma unroll
    for (int mi = 0; mi < C::MI; ++mi) a[mi] = frag((C::MI * wm + mi) * C::kFrag);
    if (kc >= 0) issue_scale(kc);
    float sgm[C::MI], sum[C::MI];  // row scale x gate / up weight scale
    auto read_scales = [&]() {
      const float sg = wsc[kb], su = wsc[kNHBlk + kb];
#pragma unroll
      for (int mi = 0; mi < C::MI; ++mi) {
        const int r = C::MI * 16 * wm + 16 * mi + lr;
        const int slot = (r / C::kScaleRowsPerWave) * kWave + r % C::kScaleRowsPerWave;
        const float sa = *(const float*)(sb + C::kSOff + slot * 4);
        sgm[mi] = sa * sg;
        sum[mi] = sa * su;
      }
    };
    // Software-pipelined over column blocks: block nj's four MFMAs are issued
    // first, then the scale FMAs of block nj - 1 (whose MFMAs have finished),
    // so the VALU work runs while the matrix core is busy; block nj + 1's B
    // fragment is read from LDS during block nj.
    v4f pp[C::MI];
#pragma unroll
    for (int nj = 0; nj < 2 * C::NJ; ++nj) {
      // two halves (row blocks 0-1, 2-3), so that only half of the previous
      // block's results are still live when this block's last MFMAs issue
      v4f pc[C::MI];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int mi = 2 * h; mi < 2 * h + 2; ++mi) pc[mi] = mfma_f8_16x16x128(bn, a[mi]);
        if (h == 0 && kc >= 0) {
#pragma unroll
          for (int q = 0; q < 2; ++q)
            if (2 * nj + q < C::kPlanesPerWave) issue_plane(kc, 2 * nj + q, nt_c);
        }
        if (h == 1 && nj + 1 < 2 * C::NJ) bn = bfrag(nj + 1);
        if (h == 1 && nj == 0) read_scales();
        if (nj > 0) {
#pragma unroll
          for (int mi = 2 * h; mi < 2 * h + 2; ++mi) {
            const float sc = nj - 1 < C::NJ ? sgm[mi] : sum[mi];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[mi][nj - 1][i] = __builtin_fmaf(pp[mi][i], sc, acc[mi][nj - 1][i]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int mi = 0; mi < C::MI; ++mi) pp[mi] = pc[mi];
    }
#pragma unroll
    for (int mi = 0; mi < C::MI; ++mi)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[mi][2 * C::NJ - 1][i] = __builtin_fmaf(pp[mi][i], sum[mi], acc[mi][2 * C::NJ - 1][i]);
  };

  // Waves whose 64 rows all lie past the tile's rows (small experts) only
  // help with the copies.
  const bool wave_live = C::MI * 16 * wm < rows;

  // Step kb: stage kb has landed (the only copy in flight) and every wave has
  // finished reading stage kb - 1, so after the barrier that buffer takes the
  // copy of stage kb + 1 while stage kb is multiplied.
  auto run = [&](auto nt_c) {
    issue(0, nt_c);
#pragma unroll 1
    for (int kb = 0; kb < kNHBlk - 1; ++kb) {
      wait_vmcnt_lgkm0<0>();
      block_barrier();
      if (wave_live)
        compute(kb, kb + 1, nt_c);
      else
        issue(kb + 1, nt_c);
    }
    wait_vmcnt_lgkm0<0>();
    block_barrier();
    if (wave_live) compute(kNHBlk - 1, -1, nt_c);
  };
  // The W13 tile of an expert that fits one row tile is read exactly once:
  // nontemporal copies, a loop of their own (a branch per copy made the
  // kernel spill).  T = 1025: GEMM1 206.6 -> 191.8 us, T = 4096 302.8 ->
  // 291.6 us; T = 8192 unchanged (its hot experts span many row tiles).
  if (X.end(e) - X.begin(e) <= C::BM)
    run(std::true_type{});
  else
    run(std::false_type{});

  // ---- SwiGLU epilogue (moe.py:190-193): act = silu(up) * gate ------------
#pragma unroll
  for (int mi = 0; mi < C::MI; ++mi) {
    const int r = C::MI * 16 * wm + 16 * mi + lr;
    if (r < rows) {
      uint16_t* arow = act + (size_t)(row0 + r) * kActRowElems;
      const int c0 = j0 + 16 * C::NJ * wn + 4 * lq;  // 4 adjacent columns: one 8-byte store per half
      // every_token_experts: the row's routing weight folded in
      const float wr = (fused >> e) & 1u ? perm_w[row0 + r] : 1.0f;
#pragma unroll
      for (int nj = 0; nj < C::NJ; ++nj) {
        float c[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) c[i] = silu_mul(acc[mi][C::NJ + nj][i], acc[mi][nj][i]);
        if ((fused >> e) & 1u) {
#pragma unroll
          for (int i = 0; i < 4; ++i) c[i] = c[i] * wr;
        }
        uint2 h, l;
        split_bf16x2(c[0], c[1], h.x, l.x);
        split_bf16x2(c[2], c[3], h.y, l.y);
        uint16_t* p = arow + act_col(c0 + 16 * nj);
        *(uint2*)p = h;
        *(uint2*)(p + 64) = l;
      }
    }
  }
  }
}

hipError_t launch_gemm1_wide(const uint8_t* hs, const float* hs_scale, int T, const uint8_t* w13,
                             const float* w13_scale, const Layout& L, char* ws, hipStream_t stream, int both) {
  using C = G1Wide;
  const int64_t pairs = (int64_t)T * kTopK;
  const int64_t mtiles = (pairs + C::BM - 1) / C::BM + (pairs < kELocal ? pairs : kELocal);
  const int64_t blocks = ((mtiles * C::kNT + 7) / 8) * 8;
  hipLaunchKernelGGL(gemm1_wide_kernel, dim3((unsigned)blocks), dim3(C::kThreads), 0, stream, hs, hs_scale, T,
                     w13, w13_scale, (const int32_t*)(ws + L.expert_off), (const int32_t*)(ws + L.perm_token),
                     (const float*)(ws + L.perm_w), (uint16_t*)(ws + L.act), both);
  return hipGetLastError();
}

}  // namespace

bool gemm1_routes(int T) { return T <= kGemm1DirectMaxTokens; }

hipError_t launch_gemm1(const uint8_t* hs, const float* hs_scale, int T, const uint8_t* w13,
                        const float* w13_scale, const float* logits, const uint16_t* bias, float rsf,
                        int64_t offset, const Layout& L, char* ws, hipStream_t stream) {
  const int32_t* off = (const int32_t*)(ws + L.expert_off);
  const int32_t* perm = (const int32_t*)(ws + L.perm_token);
  uint16_t* act = (uint16_t*)(ws + L.act);
  if (T <= kGemm1StreamMaxTokens) {
    const int max_active = min(kELocal, T * kTopK);
    if (gemm1_routes(T)) {
      const DirectRoute dr{logits, bias, rsf, offset,
                           RouteOut{(int32_t*)(ws + L.topk_ids), (float*)(ws + L.topk_w), (int32_t*)(ws + L.pair_row),
                                    (int32_t*)(ws + L.expert_off), (int32_t*)(ws + L.perm_token),
                                    (float*)(ws + L.perm_w)}};
      static ResidentGrid grid(gemm1_stream_kernel<true>, kS1Threads);
      hipLaunchKernelGGL(gemm1_stream_kernel<true>, dim3(grid.limit(max_active * kS1Groups)), dim3(kS1Threads), 0,
                         stream, hs, hs_scale, T, w13, w13_scale, off, perm, act, dr);
    } else {
      static ResidentGrid grid(gemm1_stream_kernel<false>, kS1Threads);
      hipLaunchKernelGGL(gemm1_stream_kernel<false>, dim3(grid.limit(max_active * kS1Groups)), dim3(kS1Threads), 0,
                         stream, hs, hs_scale, T, w13, w13_scale, off, perm, act, DirectRoute{});
    }
    return hipGetLastError();
  }
  if (T < kGemm1TiledLargeMinTokens) return launch_gemm1_tiled<4, 2>(hs, hs_scale, T, w13, w13_scale, L, ws, stream, 0);
  if (T <= kGemm1BothMaxTokens) {
    const hipError_t e = launch_gemm1_tiled<4, 2>(hs, hs_scale, T, w13, w13_scale, L, ws, stream, 1);
    if (e != hipSuccess) return e;
    return launch_gemm1_wide(hs, hs_scale, T, w13, w13_scale, L, ws, stream, 1);
  }
  return launch_gemm1_wide(hs, hs_scale, T, w13, w13_scale, L, ws, stream, 0);
}

}  // namespace moe
