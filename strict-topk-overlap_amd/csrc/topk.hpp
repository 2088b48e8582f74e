// Exact top-K of one row of order-preserving 64-bit keys, for a whole
// workgroup (any multiple of 64 threads).
//
// Contract: the k largest (key, -index) pairs, so ties go to the lower index,
// reported in ascending index order (the rank passed to emit()).  Method:
// MSB-first radix select with 8-bit digits starting at the highest bit where
// the row's keys differ, stopping as soon as the threshold digit's bin is
// taken whole; then block-wide scans give every selected index its rank.
// Thread t owns the contiguous indices [t*KPT, t*KPT + KPT), n <= KPT * threads.
#pragma once

#include "common.hpp"

namespace stk {

struct TopkLds {
  int hist[256];
  int tmp[16];
  uint64_t red64[2][16];
  int pick[2];
};

template <int KPT, typename EMIT>
__device__ __forceinline__ void topk_select(const uint64_t* rk, int n, int k, TopkLds& L,
                                            EMIT emit) {
  const int nwaves = blockDim.x / STK_WAVE;
  const int base = threadIdx.x * KPT;
  uint64_t key[KPT];
#pragma unroll
  for (int i = 0; i < KPT; ++i) key[i] = ld_or(rk, (int64_t)(base + i), base + i < n, (uint64_t)0);
  // bits shared by every key of the row
  uint64_t vor = 0ull, vand = ~0ull;
#pragma unroll
  for (int i = 0; i < KPT; ++i)
    if (base + i < n) {
      vor |= key[i];
      vand &= key[i];
    }
  vor = wave_or64(vor);
  vand = wave_and64(vand);
  if (lane_id() == 0) {
    L.red64[0][wave_id()] = vor;
    L.red64[1][wave_id()] = vand;
  }
  __syncthreads();
  vor = 0ull;
  vand = ~0ull;
  for (int w = 0; w < nwaves; ++w) {
    vor |= L.red64[0][w];
    vand &= L.red64[1][w];
  }
  const uint64_t diff = vor ^ vand;
  uint64_t mask = ~0ull, prefix = vand;   // when every key is equal
  int need = k;
  if (diff != 0ull) {
    int start = 63 - __clzll((long long)diff);
    mask = start == 63 ? 0ull : ~0ull << (start + 1);
    prefix = vand & mask;
    while (true) {
      const int shift = start >= 7 ? start - 7 : 0;
      const int width = start - shift + 1;
      const uint64_t dmask = ((1ull << width) - 1ull);
      for (int i = threadIdx.x; i < 256; i += blockDim.x) L.hist[i] = 0;
      __syncthreads();
#pragma unroll
      for (int i = 0; i < KPT; ++i)
        if (base + i < n && (key[i] & mask) == prefix)
          atomicAdd(&L.hist[(key[i] >> shift) & dmask], 1);
      __syncthreads();
      if (wave_id() == 0) {
        // lane l owns bins 255-4l .. 252-4l (descending digit order)
        int c[4], s = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          c[t] = L.hist[255 - 4 * lane_id() - t];
          s += c[t];
        }
        int inc = wave_incl_scan(s);
        int above = inc - s;        // keys in higher bins than this lane's
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (above < need && above + c[t] >= need) {
            L.pick[0] = 255 - 4 * lane_id() - t;
            L.pick[1] = above;
          }
          above += c[t];
        }
      }
      __syncthreads();
      const int bin = L.pick[0];
      const int above = L.pick[1];
      const int cnt = L.hist[bin];
      need -= above;
      prefix |= (uint64_t)bin << shift;
      mask |= dmask << shift;
      __syncthreads();
      if (cnt == need || shift == 0) break;
      start = shift - 1;
    }
  }
  // selected: (key & mask) > prefix, plus the `need` lowest-index keys with
  // (key & mask) == prefix
  int eq = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) eq += base + i < n && (key[i] & mask) == prefix;
  int total;
  int eq_before = block_excl_scan(eq, L.tmp, &total);
  bool sel[KPT];
  int cnt = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    bool valid = base + i < n;
    uint64_t km = key[i] & mask;
    bool e = valid && km == prefix;
    sel[i] = valid && (km > prefix || (e && eq_before < need));
    eq_before += e;
    cnt += sel[i];
  }
  int pos = block_excl_scan(cnt, L.tmp, &total);
#pragma unroll
  for (int i = 0; i < KPT; ++i)
    if (sel[i]) emit(pos++, base + i);
}

}  // namespace stk
