// route.hip -- DeepSeek-V3 grouped routing and the expert permutation, in one
// launch.
//
// Reference behaviour: moe.py:123-158 (routing) and moe.py:168-179 (per-expert
// token lists, ascending token order); the CUDA solution splits this over
// route_kernel (moe.cu:60-186), scan_offsets_kernel (moe.cu:217-265) and
// perm_fill_kernel (moe.cu:288-309, atomics, nondeterministic order).
//
// Design (gfx950, wave64):
//   * one wavefront per token, 16 tokens per 1024-thread workgroup; lane l
//     owns experts l, l+64, l+128, l+192, so a routing group of 32 experts is
//     one half-wave in one register slot;
//   * scores become 32-bit order-preserving keys; the group top-2 sums use
//     one DPP top-2 reduction per half-wave (four slots in parallel), the
//     groups are ranked one per lane, and the top-8 is a rank of the few
//     candidates at or above the kept groups' least second-largest key (DPP
//     row rotations), in expert order (route_token_lanes);
//   * T <= 24: one workgroup routes every token (a wave per token, up to two
//     tokens per wave) and builds the permutation from LDS (per-expert token
//     bitmasks), with no global atomics, fences or re-reads of the ids
//     (route_small, route_token.hpp), in one launch instead of two.  The
//     layer itself runs that routing inside GEMM1 for T <= 16; this kernel
//     serves the routing-only entry point there;
//   * larger T: each workgroup stores its local-expert histogram (plain
//     stores, no atomics); a second kernel (one workgroup per 1024 tokens)
//     reduces the histograms to the expert row offsets and the per-chunk bases
//     and scatters its chunk;
//   * ranks inside a chunk come from wave ballots, so rows of an expert are in
//     ascending token order and the result is deterministic; no host round
//     trip at any T.
#include "route_token.hpp"

namespace moe {
namespace {

constexpr int kRouteWaves = 16;      // waves per route workgroup (T > 1024: a token each)
// T <= 24: one workgroup routes and permutes every token, a wave per token
// (a second token for some waves), in one launch instead of two: T = 17
// 11.7 -> 9.4 us, T = 24 12.2 -> 10.6 us.  Beyond, a wave's routing chains
// in sequence cost more than the second launch (T = 32 +1.4 us, T = 64 +7).
constexpr int kRouteSingleMaxTokens = 24;
constexpr int kRouteWavesMulti = 4;  // tokens per route workgroup, 24 < T <= kRouteMultiSmallMaxTokens
constexpr int kRouteMultiSmallMaxTokens = 1024;
constexpr int kRouteThreads = kRouteWaves * kWave;
// Waves per permutation workgroup for 64 < T <= kRouteMultiSmallMaxTokens
// (128 tokens each, so T = 1024 takes 8 workgroups) and beyond (256 tokens
// each, 32 workgroups at T = 8192).
constexpr int kPermWavesMid = 2;
constexpr int kPermWavesLarge = 4;
static_assert((kPermWavesMid * kWave) % kRouteWavesMulti == 0, "a chunk covers whole route workgroups");
static_assert((kPermWavesLarge * kWave) % kRouteWaves == 0, "a chunk covers whole route workgroups");

// Local-expert bitmask of a token's 8 ascending ids, and the slot of its first
// local id (ids ascending => local ids occupy slots kfirst .. kfirst+popc-1).
__device__ __forceinline__ uint32_t local_mask(const int32_t id[kTopK], int64_t offset, int& kfirst) {
  uint32_t m = 0;
  kfirst = kTopK;
#pragma unroll
  for (int k = kTopK - 1; k >= 0; --k) {
    const int64_t le = (int64_t)id[k] - offset;
    if (le >= 0 && le < kELocal) {
      m |= 1u << (int)le;
      kfirst = k;
    }
  }
  return m;
}

// Shared memory of the permutation pass, for a workgroup of kPW waves.
template <int kPW>
struct PermShared {
  uint64_t wave_bal[kPW][kELocal];  // per wave and expert: ballot of the lanes (tokens) that pick it
  int wave_cnt[kPW][kELocal];
  int wave_base[kPW][kELocal];
  int running[kELocal];  // next free row per expert
  int total[kELocal];    // pairs per expert (all tokens)
  int before[kELocal];   // pairs per expert in tokens before this chunk
};

// Writes expert_off (when `write_off`) and sets running[e] = expert_off[e] +
// before[e] from the totals in shared memory.  Called by wave 0.
template <int kPW>
__device__ __forceinline__ void expert_offsets(PermShared<kPW>& sh, bool write_off, int32_t* __restrict__ expert_off) {
  const int lane = threadIdx.x & (kWave - 1);
  const int c = lane < kELocal ? sh.total[lane] : 0;
  int incl = c;
#pragma unroll
  for (int d = 1; d < kELocal; d <<= 1) {
    const int v = __shfl_up(incl, d, kWave);
    if (lane >= d) incl += v;
  }
  if (lane < kELocal) {
    sh.running[lane] = incl - c + sh.before[lane];
    if (write_off) {
      expert_off[lane] = incl - c;
      if (lane == kELocal - 1) expert_off[kELocal] = incl;
    }
  }
}

// A token's ids and weights, loaded at the start of the permutation pass so
// that their latency overlaps the histogram reduction's.
struct TokenPicks {
  int4 a, b;    // ids
  float4 u, v;  // weights
};
// Lanes past the last token load its row again (unused): a load under a
// branch would make the compiler wait for it where the branch rejoins.
__device__ __forceinline__ TokenPicks load_picks(const int32_t* __restrict__ ids, const float* __restrict__ topk_w,
                                                 int T, int t) {
  const size_t tc = (size_t)min(t, T - 1);
  TokenPicks p;
  p.a = *(const int4*)(ids + tc * kTopK);
  p.b = *(const int4*)(ids + tc * kTopK + 4);
  p.u = *(const float4*)(topk_w + tc * kTopK);
  p.v = *(const float4*)(topk_w + tc * kTopK + 4);
  return p;
}

// Rows of the pairs of tokens [t0, t0 + 64 kPW): ascending token order inside
// each expert, starting at sh.running[e].  Every thread takes part.  Each
// wave takes its 32 per-expert ballots once (lane e keeps expert e's), then
// every lane ranks only its own local picks against them (mbcnt): a loop
// over all 32 experts per pick, with the row slot chosen at run time, made
// ~2,700 instructions of one wave's serial work (T = 64: 6.5 us).
template <int kPW>
__device__ void scatter_chunk(const TokenPicks& pk, int T, int t0, int64_t offset, PermShared<kPW>& sh,
                              int32_t* __restrict__ pair_row, int32_t* __restrict__ perm_token,
                              float* __restrict__ perm_w) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int t = t0 + threadIdx.x;
  const int32_t id[kTopK] = {pk.a.x, pk.a.y, pk.a.z, pk.a.w, pk.b.x, pk.b.y, pk.b.z, pk.b.w};
  int kf = kTopK;
  uint32_t m = 0;  // tokens past T have no local expert
  if (t < T) m = local_mask(id, offset, kf);
  // lane le keeps expert le's ballot
  uint64_t mine = 0;
#pragma unroll
  for (int le = 0; le < kELocal; ++le) {
    const uint64_t b = __ballot((m >> le) & 1u);
    if (lane == le) mine = b;
  }
  if (lane < kELocal) {
    sh.wave_bal[wave][lane] = mine;
    sh.wave_cnt[wave][lane] = __popcll(mine);
  }
  __syncthreads();
  if (threadIdx.x < kELocal) {
    int acc = sh.running[threadIdx.x];
#pragma unroll
    for (int w = 0; w < kPW; ++w) {
      sh.wave_base[w][threadIdx.x] = acc;
      acc += sh.wave_cnt[w][threadIdx.x];
    }
    sh.running[threadIdx.x] = acc;
  }
  __syncthreads();
  // Row of pick k: the wave's base for its expert plus the number of lanes
  // below this one holding that expert.
  // (every pick reads the tables, at a clamped index, so that the 16 LDS
  // reads go out together instead of one wait per pick)
  int32_t row[kTopK];
  bool loc[kTopK];
  uint64_t bal[kTopK];
  int base[kTopK];
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    const int64_t le = (int64_t)id[k] - offset;
    loc[k] = t < T && le >= 0 && le < kELocal;
    const int e = loc[k] ? (int)le : 0;
    bal[k] = sh.wave_bal[wave][e];
    base[k] = sh.wave_base[wave][e];
  }
#pragma unroll
  for (int k = 0; k < kTopK; ++k) {
    const int rank =
        (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal[k] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal[k], 0u));
    row[k] = loc[k] ? base[k] + rank : -1;
  }
  if (t < T) {
    int4 r0, r1;
    r0.x = row[0]; r0.y = row[1]; r0.z = row[2]; r0.w = row[3];
    r1.x = row[4]; r1.y = row[5]; r1.z = row[6]; r1.w = row[7];
    *(int4*)(pair_row + (size_t)t * kTopK) = r0;
    *(int4*)(pair_row + (size_t)t * kTopK + 4) = r1;
    const float wv[kTopK] = {pk.u.x, pk.u.y, pk.u.z, pk.u.w, pk.v.x, pk.v.y, pk.v.z, pk.v.w};
#pragma unroll
    for (int k = 0; k < kTopK; ++k)
      if (row[k] >= 0) {
        perm_token[row[k]] = t;
        perm_w[row[k]] = wv[k];
      }
  }
  __syncthreads();  // wave_cnt / wave_base may be reused
}

// kW tokens per workgroup, one wave each.  kSingle (T <= 16): one workgroup
// of 16 waves also builds the permutation (route_small).  Otherwise every
// workgroup writes
// its per-expert counts to block_hist for perm_kernel.  Up to
// kRouteMultiSmallMaxTokens tokens the workgroups have 4 waves (one wave per
// SIMD: the routing chain of a token is a long run of dependent wave-level
// steps, which slows down when several tokens share a SIMD, and there are
// few tokens to spread); beyond, 16 (fewer histograms for perm_kernel to sum).
template <int kW, bool kSingle>
__global__ void __launch_bounds__(kW * kWave)
route_kernel(const float* __restrict__ logits, const uint16_t* __restrict__ bias, float rsf, int T,
             int64_t offset, int32_t* __restrict__ ids, float* __restrict__ w,
             int32_t* __restrict__ pair_row, int32_t* __restrict__ expert_off,
             int32_t* __restrict__ perm_token, float* __restrict__ perm_w, int32_t* __restrict__ block_hist) {
  static_assert(kW == kRouteWaves || (kW == kRouteWavesMulti && !kSingle), "route workgroup shapes");
  if constexpr (kSingle) {
    static_assert(kW == kSmallRouteMaxWaves, "the workgroup shape route_small is sized for");
    __shared__ SmallRouteT<kRouteSingleMaxTokens> sr;
    const RouteOut out{ids, w, pair_row, expert_off, perm_token, perm_w};
    route_small(logits, bias, rsf, T, offset, sr, out, true);
    return;
  }
  __shared__ int hist[kELocal];
  __shared__ uint64_t cand[kW][kRankCands];  // per wave: the top-8 candidates
  __shared__ float cand_s[kW][kRankCands];
  if (threadIdx.x < kELocal) hist[threadIdx.x] = 0;
  __syncthreads();

  const int lane = threadIdx.x & (kWave - 1);
  const int tw = threadIdx.x / kWave;
  const int t = blockIdx.x * kW + tw;
  if (t < T) {
    int e;
    float we;
    route_token_lanes(logits, bias, rsf, t, cand[tw], cand_s[tw], e, we);
    if (lane < kTopK) {
      ids[(size_t)t * kTopK + lane] = e;
      w[(size_t)t * kTopK + lane] = we;
      const int64_t le = (int64_t)e - offset;
      if (le >= 0 && le < kELocal) atomicAdd(&hist[(int)le], 1);
    }
  }
  __syncthreads();
  if (threadIdx.x < kELocal) block_hist[(size_t)blockIdx.x * kELocal + threadIdx.x] = hist[threadIdx.x];
}

// Permutation for T > 24: workgroup c of kPW waves handles tokens
// [64 kPW c, 64 kPW (c + 1)).  Every workgroup reduces the route histograms to
// the per-expert totals and to the counts of the tokens before its chunk;
// workgroup 0 writes expert_off.  The scatter's per-expert ballot loops are
// serial per wave, so the chunk is kept small up to T = 1024 (two waves, up
// to 8 workgroups: T = 1024 one 1024-thread workgroup took 8.9 us, 16 waves on
// one CU) and T <= 64 takes one wave.
template <int kPW>
__global__ void __launch_bounds__(kPW * kWave)
perm_kernel(const int32_t* __restrict__ ids, const float* __restrict__ topk_w, int T, int64_t offset,
            const int32_t* __restrict__ block_hist, int tokens_per_block, int32_t* __restrict__ pair_row,
            int32_t* __restrict__ expert_off, int32_t* __restrict__ perm_token, float* __restrict__ perm_w) {
  constexpr int kThreads = kPW * kWave;
  __shared__ PermShared<kPW> sh;
  __shared__ int4 wave_tot[kPW][kELocal / 4];
  __shared__ int4 wave_pre[kPW][kELocal / 4];
  const int nb = (T + tokens_per_block - 1) / tokens_per_block;
  const int first = blockIdx.x * (kThreads / tokens_per_block);  // route workgroups before this chunk
  const TokenPicks pk0 = load_picks(ids, topk_w, T, blockIdx.x * kThreads + threadIdx.x);
  // Histogram rows are 128 bytes: 8 threads per row, one int4 (experts
  // 4 c4 .. 4 c4 + 3) each, kRows rows per round, kBatch loads in flight per
  // thread (one wait per batch), from clamped addresses so that no load sits
  // under a branch.
  constexpr int kRows = kThreads / 8;
  constexpr int kBatch = kRows >= 64 ? 4 : 16;
  const int c4 = threadIdx.x & 7;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  int4 tot = {0, 0, 0, 0}, pre = {0, 0, 0, 0};
  for (int b0 = threadIdx.x >> 3; b0 < nb; b0 += kBatch * kRows) {
    int4 v[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      v[i] = *(const int4*)(block_hist + (size_t)min(b0 + i * kRows, nb - 1) * kELocal + 4 * c4);
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {  // masks, not branches: rows past nb or at / after this chunk
      const int b = b0 + i * kRows;
      const int mt = -(int)(b < nb), mp = mt & -(int)(b < first);
      tot.x += v[i].x & mt; tot.y += v[i].y & mt; tot.z += v[i].z & mt; tot.w += v[i].w & mt;
      pre.x += v[i].x & mp; pre.y += v[i].y & mp; pre.z += v[i].z & mp; pre.w += v[i].w & mp;
    }
  }
  // lanes l, l ^ 8, l ^ 16, ... hold the same four experts
#pragma unroll
  for (int m = 8; m < kWave; m <<= 1) {
    tot.x += __shfl_xor(tot.x, m, kWave); tot.y += __shfl_xor(tot.y, m, kWave);
    tot.z += __shfl_xor(tot.z, m, kWave); tot.w += __shfl_xor(tot.w, m, kWave);
    pre.x += __shfl_xor(pre.x, m, kWave); pre.y += __shfl_xor(pre.y, m, kWave);
    pre.z += __shfl_xor(pre.z, m, kWave); pre.w += __shfl_xor(pre.w, m, kWave);
  }
  if (lane < 8) {
    wave_tot[wave][lane] = tot;
    wave_pre[wave][lane] = pre;
  }
  // the picks are first used only here, after the histogram loads went out
  // (the compiler would otherwise use them first and wait for them alone)
  TokenPicks pk = pk0;
  asm volatile("" : "+v"(pk.a.x), "+v"(pk.a.y), "+v"(pk.a.z), "+v"(pk.a.w), "+v"(pk.b.x), "+v"(pk.b.y),
               "+v"(pk.b.z), "+v"(pk.b.w)::"memory");
  asm volatile("" : "+v"(pk.u.x), "+v"(pk.u.y), "+v"(pk.u.z), "+v"(pk.u.w), "+v"(pk.v.x), "+v"(pk.v.y),
               "+v"(pk.v.z), "+v"(pk.v.w)::"memory");
  __syncthreads();
  if (threadIdx.x < kELocal) {
    int a = 0, p = 0;
#pragma unroll
    for (int w = 0; w < kPW; ++w) {
      a += ((const int*)wave_tot[w])[threadIdx.x];
      p += ((const int*)wave_pre[w])[threadIdx.x];
    }
    sh.total[threadIdx.x] = a;
    sh.before[threadIdx.x] = p;
  }
  __syncthreads();
  if (threadIdx.x < kWave) expert_offsets(sh, blockIdx.x == 0, expert_off);
  __syncthreads();
  scatter_chunk(pk, T, blockIdx.x * kThreads, offset, sh, pair_row, perm_token, perm_w);
}

}  // namespace

hipError_t launch_route(const float* logits, const uint16_t* bias, float rsf, int T, int64_t offset,
                        const Layout& L, char* ws, hipStream_t stream) {
  int32_t* ids = (int32_t*)(ws + L.topk_ids);
  float* w = (float*)(ws + L.topk_w);
  int32_t* pair_row = (int32_t*)(ws + L.pair_row);
  int32_t* off = (int32_t*)(ws + L.expert_off);
  int32_t* perm_token = (int32_t*)(ws + L.perm_token);
  float* perm_w = (float*)(ws + L.perm_w);
  int32_t* hist = (int32_t*)(ws + L.block_hist);
  if (T <= kRouteSingleMaxTokens) {
    hipLaunchKernelGGL((route_kernel<kRouteWaves, true>), dim3(1), dim3(kRouteThreads), 0, stream, logits, bias,
                       rsf, T, offset, ids, w, pair_row, off, perm_token, perm_w, hist);
    return hipGetLastError();
  }
  const int tpb = T <= kRouteMultiSmallMaxTokens ? kRouteWavesMulti : kRouteWaves;
  const int blocks = (T + tpb - 1) / tpb;
  if (tpb == kRouteWavesMulti)
    hipLaunchKernelGGL((route_kernel<kRouteWavesMulti, false>), dim3(blocks), dim3(kRouteWavesMulti * kWave), 0,
                       stream, logits, bias, rsf, T, offset, ids, w, pair_row, off, perm_token, perm_w, hist);
  else
    hipLaunchKernelGGL((route_kernel<kRouteWaves, false>), dim3(blocks), dim3(kRouteThreads), 0, stream, logits,
                       bias, rsf, T, offset, ids, w, pair_row, off, perm_token, perm_w, hist);
  if (T <= kWave) {
    hipLaunchKernelGGL(perm_kernel<1>, dim3(1), dim3(kWave), 0, stream, (const int32_t*)ids, (const float*)w, T,
                       offset, (const int32_t*)hist, tpb, pair_row, off, perm_token, perm_w);
  } else if (T <= kRouteMultiSmallMaxTokens) {
    constexpr int kPermThreadsMid = kPermWavesMid * kWave;
    const int chunks = (T + kPermThreadsMid - 1) / kPermThreadsMid;
    hipLaunchKernelGGL(perm_kernel<kPermWavesMid>, dim3(chunks), dim3(kPermThreadsMid), 0, stream,
                       (const int32_t*)ids, (const float*)w, T, offset, (const int32_t*)hist, tpb, pair_row, off,
                       perm_token, perm_w);
  } else {
    constexpr int kPermThreadsLarge = kPermWavesLarge * kWave;
    const int chunks = (T + kPermThreadsLarge - 1) / kPermThreadsLarge;
    hipLaunchKernelGGL(perm_kernel<kPermWavesLarge>, dim3(chunks), dim3(kPermThreadsLarge), 0, stream,
                       (const int32_t*)ids, (const float*)w, T, offset, (const int32_t*)hist, tpb, pair_row, off,
                       perm_token, perm_w);
  }
  return hipGetLastError();
}

}  // namespace moe
