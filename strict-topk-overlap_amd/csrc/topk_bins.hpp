// Exact top-K of one row of order-preserving 64-bit keys by value bins, for
// a whole workgroup of full waves (the tails of the fused steps).
//
// Contract: the k largest (key, -index) pairs, so ties go to the lower index
// (the contract of topk.hpp).  Result: a bit mask per thread, bit i set when
// the thread's key i is selected; the caller ranks the selected indices.
//
// Method, built for latency (a tail is one workgroup per head, and every
// step of the selection is on its critical path):
//   A  the row's range: per-wave max / min of the keys' high 32 bits (DPP),
//      one barrier;
//   B  a 1024-bin histogram, linear in the score value over that range
//      (bin = (s - lo) * 1024 / (hi - lo) in FP32, clamped), and, up to four
//      keys per thread, the sums of its 16-bin groups: one or two LDS
//      atomics per key, one barrier;
//   C  every wave reads the whole histogram and finds the threshold bin t
//      (keys above it, keys in it) with two DPP scans, so no barrier;
//   D  if bin t is taken whole, done; otherwise its keys (a few) are listed
//      in LDS, wave 0 ranks them by (key, -index) and publishes the last one
//      taken, two barriers.
// A caller that knows a range covering the keys ahead (the one-launch
// step's tails get it with the scorers' flags) enters at B
// (topk_bins_from) and skips A's reductions and barrier.
// The bin map is monotone non-decreasing in the key (every rounding step is
// monotone, NaN keys, whose key is 0, go to bin 0), so the selection is the
// exact one whatever the ranges and roundings are.  Rows whose range is
// empty or not finite, or whose threshold bin holds more than 64 keys, take
// the radix select of topk.hpp instead (the decision is the same in every
// wave).
#pragma once

#include "topk.hpp"

namespace stk {

constexpr int kBins = 1024;
static_assert(kBins / 16 == STK_WAVE, "one 16-bin group per lane");
constexpr int kBinCands = 64;

struct TopkBinsLds {
  __align__(16) int hist[kBins];
  int grp[kBins / 16];     // sums of 16 consecutive bins (phase C reads one per lane)
  uint32_t red[2][16];     // per-wave max / min of the keys' high words
  int ncand;
  uint64_t ck[kBinCands];
  int ci[kBinCands];
  uint64_t star_key;       // the last selected key of the threshold bin
  int star_idx;            // and its index
  TopkLds radix;           // the fallback's scratch
};

// The double a key stands for, as FP32 (monotone; NaN for key 0).
__device__ __forceinline__ float key_value(uint64_t key) {
  const uint64_t b = (key >> 63) ? (key & 0x7fffffffffffffffull) : ~key;
  return (float)__longlong_as_double((long long)b);
}

template <int KPT>
__device__ __forceinline__ uint32_t topk_bins_from(const uint64_t (&key)[KPT], int n, int k,
                                                   TopkBinsLds& L, uint32_t hmax, uint32_t hmin);

// Phase A's LDS words must be free when it starts (a barrier since their
// last use).  `between` runs after barrier A and before barrier B, for the
// caller's own LDS writes that must follow a clear done before A.
template <int KPT, typename BETWEEN>
__device__ __forceinline__ uint32_t topk_bins_flags(const uint64_t (&key)[KPT], int n, int k,
                                                    TopkBinsLds& L, BETWEEN between) {
  const int nwaves = blockDim.x / STK_WAVE;
  const int base = threadIdx.x * KPT;
  const int lane = lane_id();
  // ---- A: range of the finite-or-infinite, non-NaN keys (key 0 is NaN)
  uint32_t hmax = 0u, hmin = 0xffffffffu;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const bool ok = base + i < n && key[i] != 0ull;
    const uint32_t hw = (uint32_t)(key[i] >> 32);
    hmax = ok && hw > hmax ? hw : hmax;
    hmin = ok && hw < hmin ? hw : hmin;
  }
  hmax = wave_ext_u32<true>(hmax);
  hmin = wave_ext_u32<false>(hmin);
  if (lane == 0) {
    L.red[0][wave_id()] = hmax;
    L.red[1][wave_id()] = hmin;
  }
  for (int i = threadIdx.x; i < kBins; i += blockDim.x) L.hist[i] = 0;
  if (threadIdx.x < kBins / 16) L.grp[threadIdx.x] = 0;
  if (threadIdx.x == 0) L.ncand = 0;
  __syncthreads();
  between();
  hmax = 0u;
  hmin = 0xffffffffu;
  for (int w = 0; w < nwaves; ++w) {
    hmax = L.red[0][w] > hmax ? L.red[0][w] : hmax;
    hmin = L.red[1][w] < hmin ? L.red[1][w] : hmin;
  }
  return topk_bins_from<KPT>(key, n, k, L, hmax, hmin);
}

// Phases B-D for a range [hmin, hmax] of the keys' high words known ahead
// (any range gives the exact selection; one that covers the row's keys gives
// the narrowest bins).  L.hist, L.grp and L.ncand must be zero, with a
// barrier since they were cleared and since L's last use.
template <int KPT>
__device__ __forceinline__ uint32_t topk_bins_from(const uint64_t (&key)[KPT], int n, int k,
                                                   TopkBinsLds& L, uint32_t hmax, uint32_t hmin) {
  const int base = threadIdx.x * KPT;
  const int lane = lane_id();
  // Up to four keys per thread the 16-bin group sums are kept with LDS
  // atomics during the histogram (phase C then reads one word per lane);
  // with more keys those atomics, 64 words for the whole row, contend, and
  // phase C sums its 16 bins from the histogram instead (four 16-byte reads).
  constexpr bool kGroupAtomics = KPT <= 4;
  const float lo = key_value((uint64_t)hmin << 32);
  const float hi = key_value(((uint64_t)hmax << 32) | 0xffffffffull);
  const float range = hi - lo;
  const bool binned = hmin <= hmax && range > 0.f && range <= 3.0e38f;
  uint32_t flags = 0;
  if (binned) {
    // ---- B: histogram
    const float inv = (float)kBins / range;
    int bin[KPT];
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const float x = (key_value(key[i]) - lo) * inv;   // NaN for key 0
      bin[i] = x >= (float)(kBins - 1) ? kBins - 1 : (x > 0.f ? (int)x : 0);
      if (base + i < n) {
        atomicAdd(&L.hist[bin[i]], 1);
        if constexpr (kGroupAtomics) atomicAdd(&L.grp[bin[i] >> 4], 1);
      }
    }
    __syncthreads();
    // ---- C: threshold bin, every wave alike.  Lane l takes the sum of bins
    // [kBins - 16 (l + 1), kBins - 16 l), lane 0 the top ones.
    int s;
    if constexpr (kGroupAtomics) {
      s = L.grp[kBins / 16 - 1 - lane];
    } else {
      const int4* h4 = reinterpret_cast<const int4*>(L.hist + kBins - 16 * (lane + 1));
      s = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int4 v = h4[q];
        s += (v.x + v.y) + (v.z + v.w);
      }
    }
    const int cum = wave_incl_scan_dpp(s);
    const int L16 = __ffsll((long long)__ballot(cum >= k)) - 1;
    const int above16 = __builtin_amdgcn_readlane(cum - s, L16);
    // the 16 bins of lane L16, top first, on lanes 0..15
    const int v = lane < 16 ? L.hist[kBins - 16 * L16 - 1 - lane] : 0;
    int c = v;
    c += __builtin_amdgcn_update_dpp(0, c, 0x111, 0xf, 0xf, true);
    c += __builtin_amdgcn_update_dpp(0, c, 0x112, 0xf, 0xf, true);
    c += __builtin_amdgcn_update_dpp(0, c, 0x114, 0xf, 0xf, true);
    c += __builtin_amdgcn_update_dpp(0, c, 0x118, 0xf, 0xf, true);
    const int J = __ffsll((long long)(__ballot(lane < 16 && above16 + c >= k))) - 1;
    const int t = kBins - 16 * L16 - 1 - J;
    const int cnt = __builtin_amdgcn_readlane(v, J);
    const int need = k - (above16 + __builtin_amdgcn_readlane(c, J) - cnt);
    if (cnt == need) {
#pragma unroll
      for (int i = 0; i < KPT; ++i)
        flags |= (uint32_t)(base + i < n && bin[i] >= t) << i;
      return flags;
    }
    if (cnt <= kBinCands) {
      // ---- D: rank the threshold bin's keys
#pragma unroll
      for (int i = 0; i < KPT; ++i)
        if (base + i < n && bin[i] == t) {
          const int x = atomicAdd(&L.ncand, 1);
          L.ck[x] = key[i];
          L.ci[x] = base + i;
        }
      __syncthreads();
      // wave 0 ranks them (a loop over the candidates; every wave doing it
      // would run it once per wave on each SIMD) and publishes the last one
      // taken through LDS.  With eight or more keys per thread (long rows,
      // whose threshold bins can hold tens of candidates) candidate j is read
      // by every lane from LDS, one broadcast read whose loads pipeline;
      // otherwise it comes from lane j's registers, three lane reads per
      // candidate, the form the fused steps' tails are tuned with.
      if (wave_id() == 0) {
        const uint64_t kc = lane < cnt ? L.ck[lane] : 0ull;
        const int ic = lane < cnt ? L.ci[lane] : 0x7fffffff;
        int rank = 0;
        if constexpr (KPT >= 8) {
#pragma unroll 8
          for (int j = 0; j < cnt; ++j) {
            const uint64_t kj = L.ck[j];
            const int ij = L.ci[j];
            rank += (kj > kc) || (kj == kc && ij < ic);
          }
        } else {
          for (int j = 0; j < cnt; ++j) {
            const uint32_t jh = (uint32_t)__builtin_amdgcn_readlane((int)(kc >> 32), j);
            const uint32_t jl = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)kc, j);
            const int ij = __builtin_amdgcn_readlane(ic, j);
            const uint64_t kj = ((uint64_t)jh << 32) | jl;
            rank += (kj > kc) || (kj == kc && ij < ic);
          }
        }
        if (lane < cnt && rank == need - 1) {
          L.star_key = kc;
          L.star_idx = ic;
        }
      }
      __syncthreads();
      const uint64_t ks = L.star_key;
      const int is = L.star_idx;
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        const bool sel = bin[i] > t ||
                         (bin[i] == t && (key[i] > ks || (key[i] == ks && base + i <= is)));
        flags |= (uint32_t)(base + i < n && sel) << i;
      }
      return flags;
    }
  } else {
    __syncthreads();   // as barrier B: the caller's writes in `between` are ordered
  }
  // ---- fallback: the radix select
  topk_select_keys<KPT>(key, n, k, L.radix, [&](int, int, int i) { flags |= 1u << i; });
  return flags;
}

}  // namespace stk
