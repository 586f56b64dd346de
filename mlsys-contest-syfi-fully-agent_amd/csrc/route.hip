// route.hip -- DeepSeek-V3 grouped routing and the expert permutation, in one
// launch.
//
// Reference behaviour: moe.py:123-158 (routing) and moe.py:168-179 (per-expert
// token lists, ascending token order); the CUDA solution splits this over
// route_kernel (moe.cu:60-186), scan_offsets_kernel (moe.cu:217-265) and
// perm_fill_kernel (moe.cu:288-309, atomics, nondeterministic order).
//
// Design (gfx950, wave64):
//   * one wavefront per token; lane l owns experts l, l+64, l+128, l+192, so a
//     routing group of 32 experts is one half-wave in one register slot and
//     every group reduction is a 5-step xor butterfly inside the half-wave;
//   * scores are packed into 64-bit keys (order-preserving float bits, then
//     255 - expert) so one max-reduction gives value and lowest-index
//     tie-break at once;
//   * the last workgroup to finish (device-scope counter) builds the
//     permutation: per-expert counts and ranks come from wave ballots, so rows
//     of an expert are in ascending token order and the result is
//     deterministic; no host round trip at any T.
#include "moe_common.hpp"

namespace moe {
namespace {

constexpr int kRouteTokensPerBlock = 4;  // 4 waves, one token each
constexpr int kRouteThreads = kRouteTokensPerBlock * kWave;

__device__ __forceinline__ uint64_t make_key(float v, int e) {
  return ((uint64_t)float_order_key(v) << 32) | (uint32_t)(255 - e);
}

__device__ __forceinline__ uint64_t halfwave_max(uint64_t k) {
#pragma unroll
  for (int m = 1; m < 32; m <<= 1) k = u64max(k, shfl_xor_u64(k, m));
  return k;
}

__device__ __forceinline__ uint64_t wave_max(uint64_t k) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) k = u64max(k, shfl_xor_u64(k, m));
  return k;
}

// Routes one token with one wavefront; lanes 0..7 write ids/weights.
__device__ void route_token(const float* __restrict__ logits, const uint16_t* __restrict__ bias,
                            float rsf, int t, int32_t* __restrict__ ids_out,
                            float* __restrict__ w_out) {
  const int lane = threadIdx.x & (kWave - 1);
  const int half = lane >> 5;  // 0: lanes 0-31, 1: lanes 32-63
  float s[4];
  uint64_t key[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 64 * j + lane;
    const float x = logits[(size_t)t * kEGlobal + e];
    // moe.py:127: s = 1/(1+exp(-x)); exp evaluated in double, rounded once.
    const float ex = (float)exp(-(double)x);
    s[j] = 1.0f / (1.0f + ex);
    // moe.py:128: s_with_bias = s + bias
    const float sb = s[j] + bf16_to_f32(bias[e]);
    key[j] = make_key(sb, e);
  }
  // moe.py:135-136: group score = sum of the two largest biased scores.
  // Slot j of half h holds group 2j + h.
  float gsc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint64_t k1 = halfwave_max(key[j]);
    const uint64_t k2 = halfwave_max(key[j] == k1 ? 0ull : key[j]);
    gsc[j] = float_from_order_key((uint32_t)(k1 >> 32)) + float_from_order_key((uint32_t)(k2 >> 32));
  }
  // Gather all 8 group scores into every lane.
  float G[kNGroup];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float other = __shfl_xor(gsc[j], 32, kWave);
    G[2 * j] = half ? other : gsc[j];
    G[2 * j + 1] = half ? gsc[j] : other;
  }
  // moe.py:139-146: keep the top-4 groups (ties -> lower group index).
  uint32_t keep = 0;
#pragma unroll
  for (int g = 0; g < kNGroup; ++g) {
    int rank = 0;
#pragma unroll
    for (int h = 0; h < kNGroup; ++h) rank += (G[h] > G[g]) || (G[h] == G[g] && h < g);
    keep |= (rank < kTopKGroup ? 1u : 0u) << g;
  }
  // moe.py:149-151: top-8 experts among the kept groups.
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (!((keep >> (2 * j + half)) & 1u)) key[j] = 0ull;
  int sel[kTopK];
#pragma unroll
  for (int r = 0; r < kTopK; ++r) {
    uint64_t m = u64max(u64max(key[0], key[1]), u64max(key[2], key[3]));
    m = wave_max(m);
    const int e = 255 - (int)(uint32_t)(m & 0xFFu);
    sel[r] = e;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (key[j] == m) key[j] = 0ull;
  }
  // Sort the 8 ids ascending (uniform across the wave).
#pragma unroll
  for (int a = 1; a < kTopK; ++a)
#pragma unroll
    for (int b = kTopK - 1; b >= a; --b)
      if (sel[b - 1] > sel[b]) {
        const int tmp = sel[b];
        sel[b] = sel[b - 1];
        sel[b - 1] = tmp;
      }
  // moe.py:154-158: weights from the un-biased sigmoid, summed in ascending id
  // order, normalised (true division) then scaled.
  float sv[kTopK];
  float sum = 0.0f;
#pragma unroll
  for (int r = 0; r < kTopK; ++r) {
    const int e = sel[r];
    const int j = e >> 6;
    const float mine = j == 0 ? s[0] : j == 1 ? s[1] : j == 2 ? s[2] : s[3];
    sv[r] = __shfl(mine, e & 63, kWave);
    sum = sum + sv[r];
  }
  const float denom = sum + 1e-20f;
  if (lane < kTopK) {
    float mys = sv[0];
    int mye = sel[0];
#pragma unroll
    for (int r = 1; r < kTopK; ++r)
      if (lane == r) {
        mys = sv[r];
        mye = sel[r];
      }
    ids_out[(size_t)t * kTopK + lane] = mye;
    w_out[(size_t)t * kTopK + lane] = (mys / denom) * rsf;
  }
}

// Local-expert bitmask of token t and the position of its first local id.
__device__ __forceinline__ uint32_t local_mask(const int32_t* __restrict__ ids, int t,
                                               int64_t offset, int& kfirst) {
  uint32_t m = 0;
  kfirst = kTopK;
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    const int64_t le = (int64_t)ids[(size_t)t * kTopK + k] - offset;
    if (le >= 0 && le < kELocal) {
      m |= 1u << (int)le;
      kfirst = min(kfirst, k);
    }
  }
  return m;
}

// Executed by the last route workgroup: expert row offsets, permutation and
// pair -> row map, deterministic (ascending token order inside each expert).
__device__ void build_permutation(const int32_t* __restrict__ ids, int T, int64_t offset,
                                  int32_t* __restrict__ pair_row, int32_t* __restrict__ expert_off,
                                  int32_t* __restrict__ perm_token) {
  constexpr int kWaves = kRouteThreads / kWave;
  __shared__ int wave_cnt[kWaves][kELocal];
  __shared__ int running[kELocal];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));

  // Pass 1: per-expert counts.  Each wave accumulates its own row.
  if (lane < kELocal) wave_cnt[wave][lane] = 0;
  __syncthreads();
  for (int base = 0; base < T; base += kRouteThreads) {
    const int t = base + threadIdx.x;
    int kf;
    const uint32_t m = t < T ? local_mask(ids, t, offset, kf) : 0u;
#pragma unroll 4
    for (int le = 0; le < kELocal; ++le) {
      const uint64_t b = __ballot((m >> le) & 1u);
      if (lane == 0) wave_cnt[wave][le] += __popcll(b);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int le = 0; le < kELocal; ++le) {
      int n = 0;
      for (int w = 0; w < kWaves; ++w) n += wave_cnt[w][le];
      expert_off[le] = acc;
      running[le] = acc;
      acc += n;
    }
    expert_off[kELocal] = acc;
  }
  __syncthreads();

  // Pass 2: ranks -> rows.
  for (int base = 0; base < T; base += kRouteThreads) {
    const int t = base + threadIdx.x;
    int kf = kTopK;
    const uint32_t m = t < T ? local_mask(ids, t, offset, kf) : 0u;
#pragma unroll 4
    for (int le = 0; le < kELocal; ++le) {
      const uint64_t b = __ballot((m >> le) & 1u);
      if (lane == 0) wave_cnt[wave][le] = __popcll(b);
    }
    __syncthreads();
    // Lanes past T have m == 0: they take part in the ballots and write nothing.
    int j = 0;  // j-th local id of this token (its ids are ascending)
    for (int le = 0; le < kELocal; ++le) {
      const uint64_t b = __ballot((m >> le) & 1u);
      if ((m >> le) & 1u) {
        int row = running[le] + __popcll(b & lt_mask);
        for (int w = 0; w < wave; ++w) row += wave_cnt[w][le];
        pair_row[(size_t)t * kTopK + kf + j] = row;
        perm_token[row] = t;
        ++j;
      }
    }
    if (t < T) {
#pragma unroll
      for (int k = 0; k < kTopK; ++k)
        if (k < kf || k >= kf + j) pair_row[(size_t)t * kTopK + k] = -1;
    }
    __syncthreads();
    if (threadIdx.x < kELocal) {
      int n = 0;
      for (int w = 0; w < kWaves; ++w) n += wave_cnt[w][threadIdx.x];
      running[threadIdx.x] += n;
    }
    __syncthreads();
  }
}

__global__ void __launch_bounds__(kRouteThreads)
route_kernel(const float* __restrict__ logits, const uint16_t* __restrict__ bias, float rsf, int T,
             int64_t offset, int32_t* __restrict__ ids, float* __restrict__ w,
             int32_t* __restrict__ pair_row, int32_t* __restrict__ expert_off,
             int32_t* __restrict__ perm_token, int32_t* __restrict__ sync) {
  const int t = blockIdx.x * kRouteTokensPerBlock + threadIdx.x / kWave;
  if (t < T) route_token(logits, bias, rsf, t, ids, w);

  // Completion count; the last block builds the permutation.
  __shared__ int is_last;
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = atomicAdd(&sync[kSyncRouteDone], 1);
    is_last = (prev == (int)gridDim.x - 1);
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  build_permutation(ids, T, offset, pair_row, expert_off, perm_token);
  if (threadIdx.x == 0) sync[kSyncRouteDone] = 0;  // reusable by the next call
}

}  // namespace

hipError_t launch_route(const float* logits, const uint16_t* bias, float rsf, int T, int64_t offset,
                        const Layout& L, char* ws, hipStream_t stream) {
  const int blocks = (T + kRouteTokensPerBlock - 1) / kRouteTokensPerBlock;
  hipLaunchKernelGGL(route_kernel, dim3(blocks), dim3(kRouteThreads), 0, stream, logits, bias, rsf,
                     T, offset, (int32_t*)(ws + L.topk_ids), (float*)(ws + L.topk_w),
                     (int32_t*)(ws + L.pair_row), (int32_t*)(ws + L.expert_off),
                     (int32_t*)(ws + L.perm_token), (int32_t*)(ws + L.sync));
  return hipGetLastError();
}

}  // namespace moe
