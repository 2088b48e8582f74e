// Hybrid grouping of one query head's predicted-block states
// (strict_topk/kernels.py:94-117, _group): a block is high when its mass
// under the predicted-set softmax reaches tau times the total; the low
// blocks fold into one aggregate (m, l, u) in the frame of their largest m,
// with the absolute envelope sum |w u| beside it.
#pragma once

#include "common.hpp"

namespace stk {

struct GroupArgs {
  const float* m; const float* l; const float* u;   // states [h, s], [h, s, d]
  int h, s, d; float tau;
  uint8_t* high; float* lm; float* ll; float* lu; float* labs;
};

constexpr int kGroupRows = 256;   // state rows one workgroup groups in one round trip
constexpr int kGroupPF = 8;       // u float4s in flight per thread per pass

__device__ __forceinline__ bool group_high(float m, float l, float gm, float thr) {
  return wexp(m, gm) * l >= thr;
}

// The grouping in one memory round trip, for S <= 256 state rows, D a
// multiple of 4 (<= 1024) and 16-byte aligned rows, by one 256-thread
// workgroup: every thread issues its m, l and the u rows it will weight at
// once; the row scalars pass through LDS once, after which every wave forms
// the same global max, total mass, high flags and low frame with wave
// reductions (no further barrier); the low aggregate and its envelope are
// summed per (row group, column) and folded through LDS.
// AGENT: the states were written by other workgroups of the same launch, so
// they are read with agent-coherent loads.  POISON: the caller's wait for
// those states timed out; every output is NaN (high all 0).
template <bool AGENT>
__device__ __forceinline__ void group1_head(const GroupArgs& a, int h, bool poison = false) {
  __shared__ float s_m[kGroupRows], s_l[kGroupRows];
  __shared__ float4 s_pu[256], s_pa[256];
  const int tid = threadIdx.x, s = a.s, d = a.d;
  const float* M = a.m + (size_t)h * s;
  const float* L = a.l + (size_t)h * s;
  const float* U = a.u + (size_t)h * s * d;
  auto ldf = [](const float* p) { return AGENT ? ld_agentf(p) : *p; };
  auto ld4 = [](const float* p) {
    if constexpr (AGENT) {
      const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
      const uint64_t x0 = ld_agent(q), x1 = ld_agent(q + 1);
      return make_float4(__uint_as_float((uint32_t)x0), __uint_as_float((uint32_t)(x0 >> 32)),
                         __uint_as_float((uint32_t)x1), __uint_as_float((uint32_t)(x1 >> 32)));
    } else {
      return *reinterpret_cast<const float4*>(p);
    }
  };
  const float mv = tid < s ? ldf(M + tid) : -INFINITY;
  const float lv = tid < s ? ldf(L + tid) : 0.f;
  const int tpr = d >> 2, rgn = 256 / tpr;
  const int c4 = tid % tpr, rg = tid / tpr;
  const bool act = rg < rgn;
  const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 uu[kGroupPF];
  auto fetch = [&](int pass) {
#pragma unroll
    for (int j = 0; j < kGroupPF; ++j) {
      const int r = rg + rgn * (pass * kGroupPF + j);
      uu[j] = act && r < s ? ld4(U + (size_t)r * d + 4 * c4) : zero;
    }
  };
  fetch(0);
  s_m[tid] = mv;
  s_l[tid] = lv;
  __syncthreads();
  // ---- slot reductions, the same in every wave (lane l: rows l + 64 c)
  float pm[4], pl[4];
  float gm = -INFINITY;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int p = c * STK_WAVE + lane_id();
    pm[c] = p < s ? s_m[p] : -INFINITY;
    pl[c] = p < s ? s_l[p] : 0.f;
    gm = fmaxf(gm, pm[c]);
  }
  gm = wave_max_u(gm);
  float tot = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) tot += wexp(pm[c], gm) * pl[c];
  const float thr = a.tau * wave_sum_u(tot);
  bool hi[4];
  float lm = -INFINITY;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const bool ok = c * STK_WAVE + lane_id() < s;
    hi[c] = ok && group_high(pm[c], pl[c], gm, thr);
    lm = ok && !hi[c] ? fmaxf(lm, pm[c]) : lm;
  }
  lm = wave_max_u(lm);
  const float lowm = lm == -INFINITY ? 0.f : lm;
  float z = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const bool ok = c * STK_WAVE + lane_id() < s;
    z += ok && !hi[c] ? wexp(pm[c], lowm) * pl[c] : 0.f;
  }
  z = wave_sum_u(z);
  const float nan = __builtin_nanf("");
  if (wave_id() == 0) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int p = c * STK_WAVE + lane_id();
      if (p < s) a.high[(size_t)h * s + p] = poison ? 0 : hi[c];
    }
    if (lane_id() == 0) {
      a.lm[h] = poison ? nan : lowm;
      a.ll[h] = poison ? nan : z;
    }
  }
  // ---- low aggregate and envelope of this thread's rows
  float4 lu = zero, la = zero;
  const int passes = (s + rgn * kGroupPF - 1) / (rgn * kGroupPF);
  for (int pass = 0; pass < passes; ++pass) {
    if (pass) fetch(pass);
#pragma unroll
    for (int j = 0; j < kGroupPF; ++j) {
      const int r = rg + rgn * (pass * kGroupPF + j);
      if (act && r < s) {
        const float mr = s_m[r], lr = s_l[r];
        const float wt = group_high(mr, lr, gm, thr) ? 0.f : wexp(mr, lowm);
        const float4 x = uu[j];
        lu.x += wt * x.x; lu.y += wt * x.y; lu.z += wt * x.z; lu.w += wt * x.w;
        la.x += wt * fabsf(x.x); la.y += wt * fabsf(x.y);
        la.z += wt * fabsf(x.z); la.w += wt * fabsf(x.w);
      }
    }
  }
  s_pu[tid] = lu;
  s_pa[tid] = la;
  __syncthreads();
  if (tid < tpr) {
    float4 su = zero, sa = zero;
    for (int g = 0; g < rgn; ++g) {
      const float4 x = s_pu[g * tpr + tid], y = s_pa[g * tpr + tid];
      su.x += x.x; su.y += x.y; su.z += x.z; su.w += x.w;
      sa.x += y.x; sa.y += y.y; sa.z += y.z; sa.w += y.w;
    }
    if (poison) su = sa = make_float4(nan, nan, nan, nan);
    *reinterpret_cast<float4*>(a.lu + (size_t)h * d + 4 * tid) = su;
    *reinterpret_cast<float4*>(a.labs + (size_t)h * d + 4 * tid) = sa;
  }
}

// True when group1_head serves (s, d) with these output and state pointers.
inline bool group1_covers(int s, int d, const float* u, const float* lu, const float* labs) {
  const uintptr_t bits = reinterpret_cast<uintptr_t>(u) | reinterpret_cast<uintptr_t>(lu) |
                         reinterpret_cast<uintptr_t>(labs);
  return s <= kGroupRows && d % 4 == 0 && d <= 1024 && (bits & 15) == 0;
}

}  // namespace stk
