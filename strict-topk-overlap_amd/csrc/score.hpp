// Min/max query-sign bound scorer: the body of one scoring workgroup.
//
// Reference: strict_topk/selector.py:8-20 (_score) and strict_topk/gqa.py:15-26
// (_bound_score): score[h,n] = sum_d q_d * (q_d >= 0 ? hi : lo)[h/G, n, d].
// Evaluated in FP64: products of a 16/32-bit q and an FP32 bound are exact;
// 16 lanes share a block, lane c summing dims 64*j + 4*c + t (j ascending,
// t = 0..3) from +0.0, then an xor butterfly (8, 4, 2, 1) combines the lanes.
// A workgroup (4 waves) covers 16 * STEPS consecutive blocks of one KV head
// for all G query heads of that head, so lo/hi are read once per KV head.
#pragma once

#include "attn.hpp"

namespace stk {

constexpr int kScoreWaves = 4;

// Order-preserving map of a double to an unsigned key; NaN -> 0 (lowest),
// -0.0 -> +0.0.
__device__ __forceinline__ uint64_t score_key(double s) {
  if (s != s) return 0ull;
  if (s == 0.0) s = 0.0;
  uint64_t b = (uint64_t)__double_as_longlong(s);
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}

struct ScoreArgs {
  const void* q; int qtype;
  const float* lo; const float* hi;
  int hq, hkv, n, d;
  int chunks;            // workgroups per KV head
  float* scores;         // optional FP32 [hq, n]
  uint64_t* keys;        // optional [hq, n]
};

template <typename Q>
__device__ __forceinline__ float qval(const void* q, int64_t i) {
  return cvt(reinterpret_cast<const Q*>(q)[i]);
}

// P = 64-dim passes (D <= 64 * P), STEPS = 4-block wave steps per wave,
// GT = query heads whose rows are held in registers at a time.
template <typename Q, int P, int STEPS, bool VEC4, int GT>
__device__ __forceinline__ void score_wg(const ScoreArgs& a, int wg) {
  const int G = a.hq / a.hkv;
  const int kv = wg / a.chunks;
  const int chunk = wg % a.chunks;
  const int h0 = kv * G;
  const int lane = lane_id();
  const int lane16 = lane & 15;
  const int sub = lane >> 4;                  // block within a 4-block step
  const int wave_base = (chunk * kScoreWaves + wave_id()) * (4 * STEPS);
  const Q* qrow = reinterpret_cast<const Q*>(a.q) + (size_t)h0 * a.d;
  // every load of the wave is issued before any arithmetic, with no branch
  // around a load: out-of-range blocks, dims and heads read a valid address
  // and are zeroed
  float4 lv[STEPS][P], hv[STEPS][P];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    int nb = wave_base + 4 * s + sub;
    bool valid = nb < a.n;
    const float* lrow = a.lo + ((size_t)kv * a.n + (valid ? nb : 0)) * a.d;
    const float* hrow = a.hi + ((size_t)kv * a.n + (valid ? nb : 0)) * a.d;
#pragma unroll
    for (int j = 0; j < P; ++j) {
      int d0 = 64 * j + 4 * lane16;
      if constexpr (VEC4) {
        bool ok = valid && d0 < a.d;
        float4 l4 = *reinterpret_cast<const float4*>(lrow + (ok ? d0 : 0));
        float4 h4 = *reinterpret_cast<const float4*>(hrow + (ok ? d0 : 0));
        lv[s][j] = ok ? l4 : make_float4(0.f, 0.f, 0.f, 0.f);
        hv[s][j] = ok ? h4 : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        float l4[4], h4[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          bool ok = valid && d0 + t < a.d;
          l4[t] = ld_or(lrow, (int64_t)(d0 + t), ok, 0.f);
          h4[t] = ld_or(hrow, (int64_t)(d0 + t), ok, 0.f);
        }
        lv[s][j] = make_float4(l4[0], l4[1], l4[2], l4[3]);
        hv[s][j] = make_float4(h4[0], h4[1], h4[2], h4[3]);
      }
    }
  }
  for (int gb = 0; gb < G; gb += GT) {
    // query values of heads gb .. gb+GT-1 at this lane's dims, as doubles
    double qd[GT][P][4];
#pragma unroll
    for (int gi = 0; gi < GT; ++gi) {
      const bool hv_ok = gb + gi < G;
      const Q* qg = qrow + (size_t)(hv_ok ? gb + gi : 0) * a.d;
#pragma unroll
      for (int j = 0; j < P; ++j) {
        int d0 = 64 * j + 4 * lane16;
        if constexpr (VEC4) {
          // four consecutive elements in one 8- or 16-byte access
          bool ok = hv_ok && d0 < a.d;
          Raw<Q, 4> r;
          r.load(qg + (ok ? d0 : 0));
#pragma unroll
          for (int t = 0; t < 4; ++t) qd[gi][j][t] = ok ? (double)r.get(t) : 0.0;
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            bool ok = hv_ok && d0 + t < a.d;
            float qv = cvt(qg[ok ? d0 + t : 0]);
            qd[gi][j][t] = ok ? (double)qv : 0.0;
          }
        }
      }
    }
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int nb = wave_base + 4 * s + sub;
#pragma unroll
      for (int gi = 0; gi < GT; ++gi) {
        double acc = 0.0;
#pragma unroll
        for (int j = 0; j < P; ++j) {
          const float lvv[4] = {lv[s][j].x, lv[s][j].y, lv[s][j].z, lv[s][j].w};
          const float hvv[4] = {hv[s][j].x, hv[s][j].y, hv[s][j].z, hv[s][j].w};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            // a zero q (out of range) adds +0.0, which leaves the sum unchanged
            double b = qd[gi][j][t] >= 0.0 ? (double)hvv[t] : (double)lvv[t];
            acc = fma(qd[gi][j][t], b, acc);   // exact product, one rounding
          }
        }
        acc = acc + __shfl_xor(acc, 8);
        acc = acc + __shfl_xor(acc, 4);
        acc = acc + __shfl_xor(acc, 2);
        acc = acc + __shfl_xor(acc, 1);
        if (lane16 == 0 && nb < a.n && gb + gi < G) {
          if (acc == 0.0) acc = 0.0;
          size_t o = (size_t)(h0 + gb + gi) * a.n + nb;
          if (a.scores) a.scores[o] = (float)acc;
          if (a.keys) a.keys[o] = score_key(acc);
        }
      }
    }
  }
}


}  // namespace stk
