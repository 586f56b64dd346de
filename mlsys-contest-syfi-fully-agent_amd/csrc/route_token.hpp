// route_token.hpp -- DeepSeek-V3 grouped routing of one token by one
// wavefront (moe.py:123-158), and the whole routing with the permutation for
// up to 24 tokens in one workgroup (moe.py:168-179).  Used by the routing
// kernels and by GEMM1's decode path, which routes its few tokens itself
// instead of waiting for a routing launch.
#pragma once

#include <utility>

#include "moe_common.hpp"

namespace moe {

// Maximum over the wave, wave-uniform: DPP maxima within each row of 16
// (bound_ctrl moves, which the compiler folds into v_max_u32_dpp), then the
// four row maxima.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t k) {
  k = max(k, (uint32_t)__builtin_amdgcn_mov_dpp((int)k, kDppQuad1032, 0xF, 0xF, true));
  k = max(k, (uint32_t)__builtin_amdgcn_mov_dpp((int)k, kDppQuad2301, 0xF, 0xF, true));
  k = max(k, (uint32_t)__builtin_amdgcn_mov_dpp((int)k, kDppRowHalfMirror, 0xF, 0xF, true));
  k = max(k, (uint32_t)__builtin_amdgcn_mov_dpp((int)k, kDppRowMirror, 0xF, 0xF, true));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)k, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)k, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)k, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)k, 48);
  return max(max(a, b), max(c, d));
}

// The two largest 32-bit keys (a repeated maximum counts twice) of each
// half-wave (lanes 0-31, 32-63), wave-uniform, in one reduction: every step
// merges a lane's pair (a >= b) with a partner's.  Four DPP row steps, then
// rows 1 and 3 merge rows 0 and 2 (row_bcast:15; rows 0 and 2 merge with
// the pair (0, 0), key 0 lying below every real score).
__device__ __forceinline__ void merge_top2(uint32_t& a, uint32_t& b, uint32_t pa, uint32_t pb) {
  const uint32_t lo = min(a, pa);
  a = max(a, pa);
  b = max(max(b, pb), lo);
}
__device__ __forceinline__ void halfwave_top2(uint32_t k, uint32_t& a0, uint32_t& b0, uint32_t& a1, uint32_t& b1) {
  uint32_t a = k, b = 0u;
  merge_top2(a, b, dpp_u32<kDppQuad1032, 0xF>(a), dpp_u32<kDppQuad1032, 0xF>(b));
  merge_top2(a, b, dpp_u32<kDppQuad2301, 0xF>(a), dpp_u32<kDppQuad2301, 0xF>(b));
  merge_top2(a, b, dpp_u32<kDppRowHalfMirror, 0xF>(a), dpp_u32<kDppRowHalfMirror, 0xF>(b));
  merge_top2(a, b, dpp_u32<kDppRowMirror, 0xF>(a), dpp_u32<kDppRowMirror, 0xF>(b));
  merge_top2(a, b, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)a, kDppRowBcast15, 0xA, 0xF, false),
             (uint32_t)__builtin_amdgcn_update_dpp(0, (int)b, kDppRowBcast15, 0xA, 0xF, false));
  a0 = (uint32_t)__builtin_amdgcn_readlane((int)a, 31);
  b0 = (uint32_t)__builtin_amdgcn_readlane((int)b, 31);
  a1 = (uint32_t)__builtin_amdgcn_readlane((int)a, 63);
  b1 = (uint32_t)__builtin_amdgcn_readlane((int)b, 63);
}

// moe.py:149-151: top-8 experts among the kept groups, as eight rounds of
// (wave maximum of the keys, the lowest expert index holding it); the expert
// taken leaves the round's candidates.  This is the set "every key above the
// 8th largest, then the lowest indices among the keys equal to it" (keys of
// dropped groups must be 0, below every real score).  Lane l holds experts
// 64 j + l in slot j; the picks come out ascending.
__device__ __forceinline__ void top8_rounds(uint32_t key[4], int pick[kTopK]) {
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t taken = 0u;  // bit j: this lane's expert 64j + lane already taken
#pragma unroll
  for (int r = 0; r < kTopK; ++r) {
    const uint32_t M = wave_max_u32(max(max(key[0], key[1]), max(key[2], key[3])));
    // slot j: lanes holding M (taken experts hold 0, so only a zero maximum
    // needs the taken bits)
    uint64_t b[4];
    if (M != 0u) {
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = __ballot(key[j] == M);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = __ballot(key[j] == 0u && !((taken >> j) & 1u));
    }
    // lowest expert index 64j + lane among them
    int t = 4 * kWave;
#pragma unroll
    for (int j = 3; j >= 0; --j)
      if (b[j]) t = 64 * j + __builtin_ctzll(b[j]);
    pick[r] = t;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (64 * j + lane == t) {
        key[j] = 0u;
        taken |= 1u << j;
      }
  }
  // ids ascending: Batcher's 19-comparator network on the (wave-uniform) ids
  constexpr int kNet[19][2] = {{0, 1}, {2, 3}, {4, 5}, {6, 7}, {0, 2}, {1, 3}, {4, 6}, {5, 7}, {1, 2}, {5, 6},
                               {0, 4}, {1, 5}, {2, 6}, {3, 7}, {2, 4}, {3, 5}, {1, 2}, {3, 4}, {5, 6}};
#pragma unroll
  for (int c = 0; c < 19; ++c) {
    const int x = pick[kNet[c][0]], y = pick[kNet[c][1]];
    pick[kNet[c][0]] = min(x, y);
    pick[kNet[c][1]] = max(x, y);
  }
}

// moe.py:127-136 for token t on one wave: the un-biased scores s, the 32-bit
// keys of the biased scores, and per group the top-2 sum and the second
// largest key.
__device__ __forceinline__ void token_keys(const float* __restrict__ logits, const uint16_t* __restrict__ bias,
                                           int t, float s[4], uint32_t key[4], float G[kNGroup],
                                           uint32_t gb[kNGroup]) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 64 * j + lane;
    const float x = logits[(size_t)t * kEGlobal + e];
    // moe.py:127: s = 1/(1+exp(-x)); exp evaluated in double, rounded once.
    const float ex = (float)exp(-(double)x);
    s[j] = 1.0f / (1.0f + ex);
    // moe.py:128: s_with_bias = s + bias
    key[j] = float_order_key(s[j] + bf16_to_f32(bias[e]));
  }
  // moe.py:135-136: group score = sum of the two largest biased scores (a
  // repeated maximum counts twice).  The four slots reduce independently.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t a0, b0, a1, b1;
    halfwave_top2(key[j], a0, b0, a1, b1);
    G[2 * j] = float_from_order_key(a0) + float_from_order_key(b0);
    G[2 * j + 1] = float_from_order_key(a1) + float_from_order_key(b1);
    gb[2 * j] = b0;
    gb[2 * j + 1] = b1;
  }
}

// Routes token t with one wavefront.  Returns the 8 selected ids, ascending
// (wave-uniform), and their weights (wave-uniform).
//
// Lane l holds experts l, l+64, l+128, l+192 (slot j = expert / 64); the
// routing group of 32 experts g = 2j + (l >= 32) is one half-wave of one slot.
// Scores are compared through 32-bit order-preserving keys of the fp32 values
// (masked experts: key 0, below every real score); among equal scores the
// lower expert index wins.
__device__ inline void route_token(const float* __restrict__ logits, const uint16_t* __restrict__ bias,
                            float rsf, int t, int sel[kTopK], float wsel[kTopK]) {
  const int lane = threadIdx.x & (kWave - 1);
  float s[4];
  uint32_t key[4];
  float G[kNGroup];
  uint32_t gb[kNGroup];
  token_keys(logits, bias, t, s, key, G, gb);
  // moe.py:139-146: keep the top-4 groups (ties -> lower group index).
  uint32_t keep = 0;
#pragma unroll
  for (int g = 0; g < kNGroup; ++g) {
    int rank = 0;
#pragma unroll
    for (int h = 0; h < kNGroup; ++h) rank += (G[h] > G[g]) || (G[h] == G[g] && h < g);
    keep |= (rank < kTopKGroup ? 1u : 0u) << g;
  }
  const int half = lane >> 5;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (!((keep >> (2 * j + half)) & 1u)) key[j] = 0u;
  int pick[kTopK];
  top8_rounds(key, pick);
#pragma unroll
  for (int r = 0; r < kTopK; ++r) {
    const int j = pick[r] >> 6, l = pick[r] & 63;
    sel[r] = pick[r];
    const float sj = j == 0 ? s[0] : j == 1 ? s[1] : j == 2 ? s[2] : s[3];
    wsel[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sj), l));
  }
  // moe.py:154-158: weights from the un-biased sigmoid, summed in ascending id
  // order, normalised (true division) then scaled.
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < kTopK; ++k) sum = sum + wsel[k];
  const float denom = sum + 1e-20f;
#pragma unroll
  for (int k = 0; k < kTopK; ++k) wsel[k] = (wsel[k] / denom) * rsf;
}

// ---------------------------------------------------------------------------
// Routing and permutation of T <= kMaxT tokens in one workgroup, from LDS
// only (no global round trip of the ids).  Token t is routed by wave
// t % waves.  Rows of local expert le are its tokens in ascending order
// (moe.py:168-179), starting at the exclusive scan of the per-expert counts.
// `sr` is LDS of the caller (inside its single LDS object); the workspace
// outputs `out` are written only when `write_out` is set.  GEMM1's decode
// path routes up to 16 tokens this way, the routing launch up to 24.
// ---------------------------------------------------------------------------
constexpr int kSmallRouteMaxTokens = 16;
constexpr int kSmallRouteMaxWaves = 16;

template <int kMaxT>
struct SmallRouteT {
  static_assert(kMaxT <= 32, "token masks are 32 bits");
  uint32_t tokmask[kELocal];                       // bit t: token t chose local expert le
  int expert_off[kELocal + 1];                     // first row per local expert; [32] = rows
  int pair_id[kMaxT][kTopK];                       // selected global ids, ascending
  float pair_w[kMaxT][kTopK];                      // their weights
  int perm_token[kMaxT * kTopK];                   // token of each permuted row
  float perm_w[kMaxT * kTopK];                     // weight of each permuted row
  // T == 1 (route_one): the token's 32-bit keys, sigmoid scores, group scores,
  // each group's second largest key, and the compacted top-8 candidates
  uint32_t key1[kEGlobal];
  float s1[kEGlobal];
  float g1[kNGroup];
  uint32_t gb1[kNGroup];
  uint64_t cand[16];
  // T >= 2 (route_token_lanes, a wave per token): each wave's top-8 candidates
  uint64_t cand_w[kSmallRouteMaxWaves][16];
  float cand_sw[kSmallRouteMaxWaves][16];
};
using SmallRoute = SmallRouteT<kSmallRouteMaxTokens>;

struct RouteOut {
  int32_t* ids;
  float* w;
  int32_t* pair_row;
  int32_t* expert_off;
  int32_t* perm_token;
  float* perm_w;
};

// The top-8 as a rank rather than eight rounds of a wave maximum (one wave's
// serial chain of ~240 dependent instructions, 1.5 us of the decode layer):
// each kept group's two largest keys are eight candidates, so the
// 8th-largest key is at least tau, the least of the kept groups' second
// largest keys.  The keys >= tau (about a dozen) are compacted in expert
// order into LDS, each lane ranks one of them against all by (key, then
// lower expert), and the ranks below 8 are the picks, already in ascending
// expert order.  More than kRankCands candidates take the eight rounds.
constexpr int kRankCands = 16;
static_assert(kRankCands == 16, "one DPP row of candidates; SmallRoute sizes its scratch for 16");

// Set bits of a wave mask below this lane (mbcnt).
__device__ __forceinline__ int lane_rank(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// 1 where lane (l + K) % 16 of l's DPP row holds a larger 64-bit value than l
// (row_ror:K), else 0.
template <int K>
__device__ __forceinline__ int row_ror_greater(uint32_t lo, uint32_t hi, uint64_t v) {
  const uint32_t l = (uint32_t)__builtin_amdgcn_mov_dpp((int)lo, 0x120 + K, 0xF, 0xF, true);
  const uint32_t h = (uint32_t)__builtin_amdgcn_mov_dpp((int)hi, 0x120 + K, 0xF, 0xF, true);
  return (((uint64_t)h << 32) | l) > v ? 1 : 0;
}
template <int... K>
__device__ __forceinline__ int row_rank_greater(uint32_t lo, uint32_t hi, uint64_t v,
                                                std::integer_sequence<int, K...>) {
  return (row_ror_greater<K + 1>(lo, hi, v) + ...);
}

// route_token with the result per lane (lane r < 8: pick r, ascending, and
// its weight) and the top-8 found as route_one does: the groups are ranked
// one per lane, the kept groups' keys at or above tau (the least of their
// second largest keys) are compacted in expert order into `cand` / `cs`
// (16 entries of this wave's LDS) and ranked against each other by DPP row
// rotations, and each of lanes 0-7 divides its own weight.  More than 16
// candidates, fewer than four kept groups (NaN scores) or a kept key of 0
// take the eight rounds.  Same results as route_token, bit for bit.
__device__ inline void route_token_lanes(const float* __restrict__ logits, const uint16_t* __restrict__ bias,
                                         float rsf, int t, uint64_t* cand, float* cs, int& pick_l, float& w_l) {
  const int lane = threadIdx.x & (kWave - 1);
  float s[4];
  uint32_t key[4];
  float G[kNGroup];
  uint32_t gb[kNGroup];
  token_keys(logits, bias, t, s, key, G, gb);
  // moe.py:139-146: keep the top-4 groups (ties -> lower group index);
  // lane g < 8 ranks group g
  const int gl = lane & (kNGroup - 1);
  float Gl = G[0];
  uint32_t gbl = gb[0];
#pragma unroll
  for (int g = 1; g < kNGroup; ++g) {
    Gl = gl == g ? G[g] : Gl;
    gbl = gl == g ? gb[g] : gbl;
  }
  int grank = 0;
#pragma unroll
  for (int h = 0; h < kNGroup; ++h) grank += (G[h] > Gl) || (G[h] == Gl && h < gl);
  const uint32_t keep = (uint32_t)__ballot(lane < kNGroup && grank < kTopKGroup) & ((1u << kNGroup) - 1u);
  const int half = lane >> 5;
  bool kept[4], zero = false;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    kept[j] = (keep >> (2 * j + half)) & 1u;
    zero |= kept[j] && key[j] == 0u;
  }
  float s_l = 0.0f;
  bool ranked = false;
  if (__popc(keep) == kTopKGroup && !__ballot(zero)) {
    uint32_t tm = (keep >> gl) & 1u ? gbl : ~0u;
    tm = min(tm, dpp_u32<kDppQuad1032, 0xF>(tm));
    tm = min(tm, dpp_u32<kDppQuad2301, 0xF>(tm));
    tm = min(tm, dpp_u32<kDppRowHalfMirror, 0xF>(tm));
    const uint32_t tau = (uint32_t)__builtin_amdgcn_readlane((int)tm, 0);
    uint64_t c[4];
    int base[5];
    base[0] = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c[j] = __ballot(kept[j] && key[j] >= tau);
      base[j + 1] = base[j] + __popcll(c[j]);
    }
    const int n = base[4];
    if (n <= kRankCands) {
      // moe.py:149-151 as a rank over (key, 255 - expert), positions in
      // expert order (slot-major, then lane)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (kept[j] && key[j] >= tau) {
          const int pos = base[j] + lane_rank(c[j]);
          cand[pos] = ((uint64_t)key[j] << 32) | (uint32_t)(255 - (64 * j + lane));
          cs[pos] = s[j];
        }
      const uint64_t v = lane < n ? cand[lane] : 0;
      const float sv = lane < n ? cs[lane] : 0.0f;
      const int rank = row_rank_greater((uint32_t)v, (uint32_t)(v >> 32), v,
                                        std::make_integer_sequence<int, kRankCands - 1>{});
      const bool chosen = lane < n && rank < kTopK;
      const int dst = (chosen ? lane_rank(__ballot(chosen)) : kWave - 1) * 4;
      pick_l = __builtin_amdgcn_ds_permute(dst, 255 - (int)(uint32_t)v);
      s_l = __builtin_bit_cast(float, __builtin_amdgcn_ds_permute(dst, __builtin_bit_cast(int, sv)));
      ranked = true;
    }
  }
  if (!ranked) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (!kept[j]) key[j] = 0u;
    int pick[kTopK];
    top8_rounds(key, pick);
    pick_l = pick[0];
#pragma unroll
    for (int r = 0; r < kTopK; ++r) {
      const int j = pick[r] >> 6, l = pick[r] & 63;
      const float sj = j == 0 ? s[0] : j == 1 ? s[1] : j == 2 ? s[2] : s[3];
      const float sr_ = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sj), l));
      if (gl == r) {
        pick_l = pick[r];
        s_l = sr_;
      }
    }
  }
  // moe.py:154-158: un-biased scores summed in ascending id order,
  // normalised (true division) then scaled; lane r divides weight r
  float sum = 0.0f;
#pragma unroll
  for (int r = 0; r < kTopK; ++r) sum = sum + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s_l), r));
  w_l = (s_l / (sum + 1e-20f)) * rsf;
}

// T == 1: the same routing as route_token, with the work of one token spread
// over four waves (waves 0-3 each compute one 64-expert slot's keys and its
// two group scores) and the top-8 (as a rank, above) over the 128 experts of
// the kept groups only (two keys per lane in wave 0), then the permutation
// of the single token written directly.  Needs at least 4 waves; ends with
// a workgroup barrier.
template <int kMaxT>
__device__ inline void route_one(const float* __restrict__ logits, const uint16_t* __restrict__ bias, float rsf,
                                 int64_t offset, SmallRouteT<kMaxT>& sr, RouteOut out, bool write_out) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  if (wave < 4) {
    const int e = 64 * wave + lane;
    const float x = logits[e];
    // moe.py:127-128 (as route_token): exp in double, rounded once; biased score
    const float ex = (float)exp(-(double)x);
    const float sv = 1.0f / (1.0f + ex);
    const uint32_t key = float_order_key(sv + bf16_to_f32(bias[e]));
    sr.s1[e] = sv;
    sr.key1[e] = key;
    // moe.py:135-136: the slot's two groups (half-waves), top-2 sums
    uint32_t a0, b0, a1, b1;
    halfwave_top2(key, a0, b0, a1, b1);
    if (lane == 0) {
      sr.g1[2 * wave] = float_from_order_key(a0) + float_from_order_key(b0);
      sr.g1[2 * wave + 1] = float_from_order_key(a1) + float_from_order_key(b1);
      sr.gb1[2 * wave] = b0;
      sr.gb1[2 * wave + 1] = b1;
    }
  }
  __syncthreads();
  if (wave == 0) {
    // moe.py:139-146: keep the top-4 groups (ties -> lower group index);
    // lane g < 8 ranks group g
    const int gl = lane & (kNGroup - 1);
    const float Gl = sr.g1[gl];
    const uint32_t gbl = sr.gb1[gl];
    int grank = 0;
#pragma unroll
    for (int h = 0; h < kNGroup; ++h) {
      const float Gh = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, Gl), h));
      grank += (Gh > Gl) || (Gh == Gl && h < gl);
    }
    const uint32_t keep = (uint32_t)__ballot(lane < kNGroup && grank < kTopKGroup) & ((1u << kNGroup) - 1u);
    // Candidates: lane l holds expert 32 kg[l/32] + l%32 (slot 0) and
    // 32 kg[2 + l/32] + l%32 (slot 1), kg the kept groups ascending, so
    // (slot, lane) order is expert order.  Exactly four groups are kept
    // unless group scores are NaN; then, and when a kept key is 0 (the key
    // route_token gives dropped experts), route_token's own selection runs.
    int kg[kTopKGroup];
    uint32_t m = keep;
#pragma unroll
    for (int k = 0; k < kTopKGroup; ++k) {
      kg[k] = m ? __builtin_ctz(m) : 0;
      m &= m - 1;
    }
    const int half = lane >> 5;
    const int ea = 32 * (half ? kg[1] : kg[0]) + (lane & 31), eb = 32 * (half ? kg[3] : kg[2]) + (lane & 31);
    uint32_t key[2] = {sr.key1[ea], sr.key1[eb]};
    const bool plain = __popc(keep) == kTopKGroup && !__ballot(key[0] == 0u || key[1] == 0u);
    // pick_l: lane r < 8 receives the r-th pick (ascending expert id)
    int pick_l = 0;
    bool ranked = false;
    if (plain) {
      // tau: minimum over lanes 0-7 (row 0's first half) of the kept
      // groups' second largest keys
      uint32_t t = (keep >> gl) & 1u ? gbl : ~0u;
      t = min(t, dpp_u32<kDppQuad1032, 0xF>(t));
      t = min(t, dpp_u32<kDppQuad2301, 0xF>(t));
      t = min(t, dpp_u32<kDppRowHalfMirror, 0xF>(t));
      const uint32_t tau = (uint32_t)__builtin_amdgcn_readlane((int)t, 0);
      const uint64_t c0 = __ballot(key[0] >= tau), c1 = __ballot(key[1] >= tau);
      const int n0 = __popcll(c0), n = n0 + __popcll(c1);
      if (n <= kRankCands) {
        // moe.py:149-151 as a rank: (key, 255 - expert) orders the
        // candidates as the selection does (larger key first, then the
        // lower expert); positions follow expert order
        if (key[0] >= tau) sr.cand[lane_rank(c0)] = ((uint64_t)key[0] << 32) | (uint32_t)(255 - ea);
        if (key[1] >= tau) sr.cand[n0 + lane_rank(c1)] = ((uint64_t)key[1] << 32) | (uint32_t)(255 - eb);
        // lanes 0-15 (one DPP row) hold the candidates, lanes n.. of the row
        // 0, which ranks below every candidate (keys >= tau > 0)
        const uint64_t v = lane < n ? sr.cand[lane] : 0;
        const int rank = row_rank_greater((uint32_t)v, (uint32_t)(v >> 32), v,
                                          std::make_integer_sequence<int, kRankCands - 1>{});
        const bool chosen = lane < n && rank < kTopK;
        const uint64_t selm = __ballot(chosen);  // exactly 8: the ranks are distinct
        // a chosen candidate goes to the lane of its place in expert order
        // (the others to lane 63, which is never read)
        pick_l = __builtin_amdgcn_ds_permute((chosen ? lane_rank(selm) : kWave - 1) * 4, 255 - (int)(uint32_t)v);
        ranked = true;
      }
    }
    if (!ranked) {
      int pick[kTopK];
      if (plain) {
        // moe.py:149-151: eight rounds of (wave maximum, lowest expert holding it)
#pragma unroll
        for (int r = 0; r < kTopK; ++r) {
          const uint32_t M = wave_max_u32(max(key[0], key[1]));
          const uint64_t b0 = __ballot(key[0] == M), b1 = __ballot(key[1] == M);
          const int l = b0 ? __builtin_ctzll(b0) : __builtin_ctzll(b1);
          const int slot = b0 ? 0 : 1;
          const int hl = l >> 5;
          pick[r] = 32 * (slot ? (hl ? kg[3] : kg[2]) : (hl ? kg[1] : kg[0])) + (l & 31);
          if (lane == l) key[slot] = 0u;  // taken (no candidate key is 0)
        }
        constexpr int kNet[19][2] = {{0, 1}, {2, 3}, {4, 5}, {6, 7}, {0, 2}, {1, 3}, {4, 6}, {5, 7}, {1, 2}, {5, 6},
                                     {0, 4}, {1, 5}, {2, 6}, {3, 7}, {2, 4}, {3, 5}, {1, 2}, {3, 4}, {5, 6}};
#pragma unroll
        for (int c = 0; c < 19; ++c) {
          const int x0 = pick[kNet[c][0]], y0 = pick[kNet[c][1]];
          pick[kNet[c][0]] = min(x0, y0);
          pick[kNet[c][1]] = max(x0, y0);
        }
      } else {
        float wsel[kTopK];  // the same weights as computed below (same scores, same order)
        route_token(logits, bias, rsf, 0, pick, wsel);
      }
#pragma unroll
      for (int r = 0; r < kTopK; ++r) pick_l = (lane & (kTopK - 1)) == r ? pick[r] : pick_l;
    }
    pick_l &= kEGlobal - 1;  // lanes past 8 hold no pick
    // moe.py:154-158: un-biased scores, summed in ascending id order,
    // normalised (true division) then scaled -- as route_token; lane r
    // divides weight r
    const float s_l = sr.s1[pick_l];
    float sum = 0.0f;
#pragma unroll
    for (int r = 0; r < kTopK; ++r) sum = sum + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s_l), r));
    const float w_l = (s_l / (sum + 1e-20f)) * rsf;
    // moe.py:168-179 for one token: its local experts, ascending, take rows
    // 0, 1, ...; expert_off[le] counts the local picks below le
    const int64_t le = (int64_t)pick_l - offset;
    const bool loc = lane < kTopK && le >= 0 && le < kELocal;
    const int row = loc ? lane_rank(__ballot(loc)) : -1;
    uint32_t lm = 0u;  // bit le: local expert le is picked
#pragma unroll
    for (int r = 0; r < kTopK; ++r) lm |= (uint32_t)__builtin_amdgcn_readlane(loc ? (int)(1u << (int)le) : 0, r);
    if (lane <= kELocal) {
      const int below = __popc((uint32_t)((uint64_t)lm & ((1ull << lane) - 1ull)));
      sr.expert_off[lane] = below;
      if (write_out) out.expert_off[lane] = below;
      if (lane < kELocal) sr.tokmask[lane] = (lm >> lane) & 1u;
    }
    if (lane < kTopK) {
      sr.pair_id[0][lane] = pick_l;
      sr.pair_w[0][lane] = w_l;
      if (row >= 0) {
        sr.perm_token[row] = 0;
        sr.perm_w[row] = w_l;
      }
      if (write_out) {
        out.ids[lane] = pick_l;
        out.w[lane] = w_l;
        out.pair_row[lane] = row;
        if (row >= 0) {
          out.perm_token[row] = 0;
          out.perm_w[row] = w_l;
        }
      }
    }
  }
  __syncthreads();
}

template <int kMaxT>
__device__ inline void route_small(const float* __restrict__ logits, const uint16_t* __restrict__ bias, float rsf,
                                   int T, int64_t offset, SmallRouteT<kMaxT>& sr, RouteOut out, bool write_out) {
  if (T == 1) {
    route_one(logits, bias, rsf, offset, sr, out, write_out);
    return;
  }
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int waves = blockDim.x / kWave;
  if (threadIdx.x < kELocal) sr.tokmask[threadIdx.x] = 0u;
  __syncthreads();
  for (int t = wave; t < T; t += waves) {
    int e;
    float we;
    route_token_lanes(logits, bias, rsf, t, sr.cand_w[wave], sr.cand_sw[wave], e, we);
    if (lane < kTopK) {
      if (write_out) {
        out.ids[(size_t)t * kTopK + lane] = e;
        out.w[(size_t)t * kTopK + lane] = we;
      }
      sr.pair_id[t][lane] = e;
      sr.pair_w[t][lane] = we;
      const int64_t le = (int64_t)e - offset;
      if (le >= 0 && le < kELocal) atomicOr(&sr.tokmask[(int)le], 1u << t);
    }
  }
  __syncthreads();
  if (threadIdx.x < kWave) {
    const int c = lane < kELocal ? __popc(sr.tokmask[lane]) : 0;
    int incl = c;
#pragma unroll
    for (int d = 1; d < kELocal; d <<= 1) {
      const int v = __shfl_up(incl, d, kWave);
      if (lane >= d) incl += v;
    }
    if (lane < kELocal) {
      sr.expert_off[lane] = incl - c;
      if (write_out) out.expert_off[lane] = incl - c;
      if (lane == kELocal - 1) {
        sr.expert_off[kELocal] = incl;
        if (write_out) out.expert_off[kELocal] = incl;
      }
    }
  }
  __syncthreads();
  for (int p = threadIdx.x; p < T * kTopK; p += blockDim.x) {  // pair p = (token p / 8, slot p % 8)
    const int pt = p / kTopK, k = p % kTopK;
    const int64_t le = (int64_t)sr.pair_id[pt][k] - offset;
    int row = -1;
    if (le >= 0 && le < kELocal) {
      row = sr.expert_off[le] + __popc(sr.tokmask[le] & ((1u << pt) - 1u));
      sr.perm_token[row] = pt;
      sr.perm_w[row] = sr.pair_w[pt][k];
      if (write_out) {
        out.perm_token[row] = pt;
        out.perm_w[row] = sr.pair_w[pt][k];
      }
    }
    if (write_out) out.pair_row[p] = row;
  }
  __syncthreads();
}

}  // namespace moe
