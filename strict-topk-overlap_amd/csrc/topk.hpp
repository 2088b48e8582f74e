// Exact top-K of one row of order-preserving 64-bit keys, for a whole
// workgroup of full waves.
//
// Contract: the k largest (key, -index) pairs, so ties go to the lower index,
// reported in ascending index order (the rank passed to emit()).  Method:
// MSB-first radix select with 8-bit digits starting at the highest bit where
// the row's keys differ, stopping as soon as the threshold digit's bin is
// taken whole; then one packed block scan gives every selected index its
// rank.  Thread t owns the contiguous indices [t*KPT, t*KPT + KPT),
// n <= KPT * threads.
//
// Latency: the selection is a chain of short dependent steps, so each is
// kept short.  Histograms are double-buffered (the next pass's buffer is
// cleared behind the current one), so a pass costs two barriers; wave
// reductions and scans are DPP sequences; the final ranking is one scan.
// (LDS atomics that crowd into a few bins, as a row's keys do, cost a few
// hundred cycles per wave instruction on CDNA4, less than matching equal
// digits through ballots first.)
#pragma once

#include <type_traits>

#include "common.hpp"

namespace stk {

struct TopkLds {
  int hist[2][256];
  int pick[2][3];        // threshold bin, keys above it, keys in it
  uint64_t red[2][16];   // per-wave OR / AND of the keys
  int tmp[16];           // per-wave totals of the final scan
};

// The row's keys, thread t holding indices [t*KPT, t*KPT + KPT) (0 past n).
template <int KPT>
__device__ __forceinline__ void topk_load(const uint64_t* rk, int n, uint64_t (&key)[KPT]) {
  const int base = threadIdx.x * KPT;
#pragma unroll
  for (int i = 0; i < KPT; ++i) key[i] = ld_or(rk, (int64_t)(base + i), base + i < n, (uint64_t)0);
}

template <int KPT, typename EMIT>
__device__ __forceinline__ void topk_select_keys(const uint64_t (&key)[KPT], int n, int k,
                                                 TopkLds& L, EMIT emit) {
  const int nwaves = blockDim.x / STK_WAVE;
  const int base = threadIdx.x * KPT;
  // bits shared by every key of the row
  uint64_t vor = 0ull, vand = ~0ull;
#pragma unroll
  for (int i = 0; i < KPT; ++i)
    if (base + i < n) {
      vor |= key[i];
      vand &= key[i];
    }
  vor = wave_bits64_u<false>(vor);
  vand = wave_bits64_u<true>(vand);
  if (lane_id() == 0) {
    L.red[0][wave_id()] = vor;
    L.red[1][wave_id()] = vand;
  }
  for (int i = threadIdx.x; i < 256; i += blockDim.x) L.hist[0][i] = 0;
  __syncthreads();
  vor = 0ull;
  vand = ~0ull;
  for (int w = 0; w < nwaves; ++w) {
    vor |= L.red[0][w];
    vand &= L.red[1][w];
  }
  const uint64_t diff = vor ^ vand;
  uint64_t mask = ~0ull, prefix = vand;   // when every key is equal
  int need = k;
  if (diff != 0ull) {
    int start = 63 - __clzll((long long)diff);
    mask = start == 63 ? 0ull : ~0ull << (start + 1);
    prefix = vand & mask;
    int buf = 0;
    while (true) {
      const int shift = start >= 7 ? start - 7 : 0;
      const int width = start - shift + 1;
      const uint64_t dmask = ((1ull << width) - 1ull);
#pragma unroll
      for (int i = 0; i < KPT; ++i)
        if (base + i < n && (key[i] & mask) == prefix)
          atomicAdd(&L.hist[buf][(key[i] >> shift) & dmask], 1);
      for (int i = threadIdx.x; i < 256; i += blockDim.x) L.hist[buf ^ 1][i] = 0;
      __syncthreads();
      if (wave_id() == 0) {
        // lane l owns bins 255-4l .. 252-4l (descending digit order)
        int c[4], s = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          c[t] = L.hist[buf][255 - 4 * lane_id() - t];
          s += c[t];
        }
        int above = wave_incl_scan_dpp(s) - s;   // keys in higher bins than this lane's
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (above < need && above + c[t] >= need) {
            L.pick[buf][0] = 255 - 4 * lane_id() - t;
            L.pick[buf][1] = above;
            L.pick[buf][2] = c[t];
          }
          above += c[t];
        }
      }
      __syncthreads();
      const int bin = L.pick[buf][0];
      const int cnt = L.pick[buf][2];
      need -= L.pick[buf][1];
      prefix |= (uint64_t)bin << shift;
      mask |= dmask << shift;
      if (cnt == need || shift == 0) break;
      start = shift - 1;
      buf ^= 1;
    }
  }
  // selected: (key & mask) > prefix, plus the `need` lowest-index keys with
  // (key & mask) == prefix; one scan of (above, equal) counts packed in 16-bit
  // halves (n <= 65535) ranks both
  int gt = 0, eq = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const bool valid = base + i < n;
    const uint64_t km = key[i] & mask;
    gt += valid && km > prefix;
    eq += valid && km == prefix;
  }
  int total;
  const int pre = block_excl_scan1(gt | (eq << 16), L.tmp, &total);
  int eq_before = pre >> 16;
  int pos = (pre & 0xffff) + min(eq_before, need);
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const bool valid = base + i < n;
    const uint64_t km = key[i] & mask;
    const bool e = valid && km == prefix;
    const bool sel = valid && (km > prefix || (e && eq_before < need));
    eq_before += e;
    if (sel) {
      // emit(rank, index) or emit(rank, index, i): i is the key's slot in
      // this thread's registers (a compile-time index once unrolled)
      if constexpr (std::is_invocable_v<EMIT, int, int, int>) emit(pos++, base + i, i);
      else emit(pos++, base + i);
    }
  }
}

// Load the row at rk and select from it.
template <int KPT, typename EMIT>
__device__ __forceinline__ void topk_select(const uint64_t* rk, int n, int k, TopkLds& L,
                                            EMIT emit) {
  uint64_t key[KPT];
  topk_load<KPT>(rk, n, key);
  topk_select_keys<KPT>(key, n, k, L, emit);
}

}  // namespace stk
