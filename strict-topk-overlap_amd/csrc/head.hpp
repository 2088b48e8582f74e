// Per-head workgroup building blocks used by the repair kernels.
//
// A repair workgroup owns one query head: 256 threads = 4 waves.  ID rows are
// staged in LDS as int64; the hit/miss partition is an equality join over the
// two rows (brute force, the reference computes the same P x A matrix,
// strict_topk/kernels.py:129, fused.py:64).  Weighted sums of saved states
// use RG row groups x DT dim threads; lists of blocks are streamed by the 4
// waves in parallel with the Tile routine and combined in LDS.
#pragma once

#include "attn.hpp"

namespace stk {

constexpr int kMaxIds = 4096;   // per-row ID capacity of the per-head kernels
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / STK_WAVE;

struct HeadLds {
  int64_t a[kMaxIds];
  int64_t p[kMaxIds];
  uint8_t fa[kMaxIds];    // per selected position flags
  uint8_t fp[kMaxIds];    // per predicted position flags
  float red[32];
  int ired[32];
  float u0[kMaxD];        // D-vector accumulators
  float u1[kMaxD];
  float u2[kMaxD];
  float part[kThreads * 4];
  float wm[kWaves];
  float wl[kWaves];
  float wu[kWaves][kMaxD];
};

__device__ __forceinline__ void stage_ids(const void* ids, int itype, int64_t base, int n,
                                          int64_t* dst) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) dst[i] = load_id(ids, itype, base + i);
}

// hit[p] = P[p] in A (into fp), miss[a] = A[a] not in P (into fa).
__device__ __forceinline__ void membership(HeadLds& s, int sp, int sa) {
  for (int i = threadIdx.x; i < sp; i += blockDim.x) {
    int64_t x = s.p[i];
    uint8_t f = 0;
    for (int j = 0; j < sa; ++j) f |= (s.a[j] == x);
    s.fp[i] = f;
  }
  for (int i = threadIdx.x; i < sa; i += blockDim.x) {
    int64_t x = s.a[i];
    uint8_t f = 0;
    for (int j = 0; j < sp; ++j) f |= (s.p[j] == x);
    s.fa[i] = !f;
  }
  __syncthreads();
}

// Weighted sum over rows j < count of (l[j], u[j,:]) with weight w(j)
// (rows with w == 0 are skipped).  Result: returned z, vector in out[D].
// A thread takes its rows four at a time: the four rows' weights, l and u
// columns are all requested before any is used (one round trip per four
// rows instead of two per row), and the sums run in the same order as one
// row at a time, so the result is the same bits.
template <typename W, typename L, typename UR>
__device__ __forceinline__ float sum_states(HeadLds& s, int count, int d, W weight, L lval,
                                            UR urow, float* out) {
  int dt = 1;
  while (dt < d && dt < kThreads) dt <<= 1;
  int rg = kThreads / dt;
  int tr = threadIdx.x / dt, td = threadIdx.x % dt;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float z = 0.f;
  constexpr int UB = 4;   // rows per batch
  for (int j0 = tr; j0 < count; j0 += UB * rg) {
    float w[UB * 2], uv[UB * 4];   // w[u] weight, w[UB + u] l
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int j = j0 + u * rg;
      const int jc = j < count ? j : j0;   // rows past count read row j0, weight 0
      const float wj = weight(jc);
      w[u] = j < count ? wj : 0.f;
      w[UB + u] = lval(jc);
      const float* ur = urow(jc);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        // columns past D read column 0; their accumulators are never read
        const int dd = td + c * dt;
        uv[4 * u + c] = ur[dd < d ? dd : 0];
      }
    }
    hold_all(w);
    hold_all(uv);
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      if (w[u] == 0.f) continue;   // a skipped row's l and u add nothing, NaN included
      if (td == 0) z += w[u] * w[UB + u];
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] += w[u] * uv[4 * u + c];
    }
  }
  z = block_sum(z, s.red);
#pragma unroll
  for (int c = 0; c < 4; ++c) s.part[c * kThreads + threadIdx.x] = acc[c];
  __syncthreads();
  for (int dd = threadIdx.x; dd < d; dd += blockDim.x) {
    int c = dd / dt, t = dd % dt;
    float sum = 0.f;
    for (int r = 0; r < rg; ++r) sum += s.part[c * kThreads + r * dt + t];
    out[dd] = sum;
  }
  __syncthreads();
  return z;
}

// Stream `count` blocks (block(j) returns the ID, or -1 to skip) through the
// 4 waves with the online softmax (or the fixed frame m_fixed when FIXED),
// and combine the wave states.  Returns (m, z) and the D-vector in out[].
// With count == 0 the result is (-inf, 0, 0) (FIXED: (m_fixed, 0, 0)).
template <typename T, int VEC, int NC, int U, bool FIXED, typename BLK>
__device__ __forceinline__ void stream_blocks(HeadLds& s, const float* qr, const Tile<T, VEC, NC>& t,
                                              const T* K, const T* V, int kv, int n, int b, int d,
                                              int count, BLK block, float m_fixed, float& m_out,
                                              float& z_out, float* out) {
  using TL = Tile<T, VEC, NC>;
  const float scale = 1.0f / sqrtf((float)d);
  float m = FIXED ? m_fixed : -INFINITY, l = 0.f, acc[TL::R];
#pragma unroll
  for (int i = 0; i < TL::R; ++i) acc[i] = 0.f;
  for (int j = wave_id(); j < count; j += kWaves) {
    int64_t bid = block(j);
    if (bid < 0 || bid >= n) continue;
    size_t off = (((size_t)kv * n + bid) * b) * d;
    t.template accum<U, FIXED, true>(qr, K + off, V + off, b, scale, m, l, acc);
  }
  t.finish(l, acc);
  if (lane_id() == 0) {
    s.wm[wave_id()] = m;
    s.wl[wave_id()] = l;
  }
  if (t.tok == 0) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      int base = (t.part + c * t.lpt) * VEC;
#pragma unroll
      for (int i = 0; i < VEC; ++i)
        if (base + i < d) s.wu[wave_id()][base + i] = acc[c * VEC + i];
    }
  }
  __syncthreads();
  float mx = s.wm[0];
  for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, s.wm[w]);
  float z = 0.f;
  float f[kWaves];
  for (int w = 0; w < kWaves; ++w) {
    f[w] = FIXED ? 1.f : wexp(s.wm[w], mx);
    z += f[w] * s.wl[w];
  }
  for (int dd = threadIdx.x; dd < d; dd += blockDim.x) {
    float sum = 0.f;
    for (int w = 0; w < kWaves; ++w) sum += f[w] * s.wu[w][dd];
    out[dd] = sum;
  }
  m_out = FIXED ? m_fixed : mx;
  z_out = z;
  __syncthreads();
}

// Exclusive-rank of set flags in position order: rank[i] for flags[i] != 0.
// Writes ranks into rk (LDS int array of n) and returns the count.
__device__ __forceinline__ int rank_flags(const uint8_t* flags, int n, int* rk, int* scan) {
  int carry = 0;
  for (int j0 = 0; j0 < n; j0 += blockDim.x) {
    int j = j0 + threadIdx.x;
    int f = (j < n) ? (flags[j] != 0) : 0;
    scan[threadIdx.x] = f;
    __syncthreads();
    for (int off = 1; off < (int)blockDim.x; off <<= 1) {
      int x = (int)threadIdx.x >= off ? scan[threadIdx.x - off] : 0;
      __syncthreads();
      scan[threadIdx.x] += x;
      __syncthreads();
    }
    if (j < n) rk[j] = carry + scan[threadIdx.x] - f;
    int tot = scan[blockDim.x - 1];
    __syncthreads();
    carry += tot;
  }
  return carry;
}

}  // namespace stk
