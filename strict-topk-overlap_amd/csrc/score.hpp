// Min/max query-sign bound scorer: the body of one scoring workgroup.
//
// Reference: strict_topk/selector.py:8-20 (_score) and strict_topk/gqa.py:15-26
// (_bound_score): score[h,n] = sum_d q_d * (q_d >= 0 ? hi : lo)[h/G, n, d].
// Evaluated in FP64: products of a 16/32-bit q and an FP32 bound are exact
// (the bounds may also be stored in the query's own 16-bit type, lb = 1:
// the min / max of 16-bit keys are 16-bit values, so that storage is exact
// and the scores are the same bits);
// 16 logical lanes share a block, lane c summing dims 64*j + 4*c + t
// (j ascending, t = 0..3) from +0.0, then an xor butterfly (8, 4, 2, 1)
// combines the lanes.  A workgroup (4 waves) covers 16 * STEPS consecutive
// blocks of one KV head for all G query heads of that head, so lo/hi are
// read once per KV head.
//
// Instruction budget (the scorer is VALU-limited once lo/hi arrive):
//   * the query heads' values are converted to FP64 once per workgroup and
//     staged in LDS with a select mask (all ones where q < 0 or q is NaN);
//   * each (head, dim, block) costs one bit-select of lo/hi, one FP32->FP64
//     conversion and one FP64 FMA;
//   * the 16-lane sums of all C = GT * STEPS (head, block) pairs of a wave
//     share one transposed reduction: at each of the first log2(C) levels a
//     lane keeps half of its pairs and adds its partner's copy of that half,
//     so the exchanges fall from 4 * C to about C.  Every exchange is a
//     single DPP move: physical lanes are permuted (score_lane) so that the
//     half-row mirror (physical xor 7) is logical xor 4; rotation by 8
//     inside a row is xor 8; quad permutations are xor 2 and xor 1.  Each
//     partial is the sum of the same two operands as in the butterfly, so
//     the bits are those of the contract.
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
  const void* lo; const void* hi;
  int lb;                // 1: lo / hi are 16-bit, the query's element type
  int hq, hkv, n, d;
  int chunks;            // workgroups per KV head
  float* scores;         // optional FP32 [hq, n]
  uint64_t* keys;        // optional [hq, n]
  uint32_t* sflag;       // SIG: [hq, fstride], entry chunk set (to the chunk's key
                         // range, never 0) once the chunk's keys are published
  int fstride;           // SIG: flag words per query head (>= chunks)
  int drop;              // SIG, tests only: publish no flag (the consumers time out)
};

// Physical lane (0..15 inside a row) -> logical lane of the summation order.
__device__ __forceinline__ int score_lane(int l16) { return l16 ^ ((l16 & 4) ? 3 : 0); }

// A DPP move of a double whose pattern reads a valid lane for every lane.
template <int CTRL>
__device__ __forceinline__ double dpp_mov_d(double v) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const int lo = __builtin_amdgcn_mov_dpp((int)(uint32_t)b, CTRL, 0xf, 0xf, false);
  const int hi = __builtin_amdgcn_mov_dpp((int)(uint32_t)(b >> 32), CTRL, 0xf, 0xf, false);
  return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}

// One halving level: keep values [0, N/2) (up = false) or [N/2, N) (up =
// true) in slots [0, N/2), adding the partner's copy of the same half.
template <int N, int CTRL>
__device__ __forceinline__ void score_halve(double* v, bool up) {
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const double keep = up ? v[N / 2 + i] : v[i];
    const double send = up ? v[i] : v[N / 2 + i];
    v[i] = keep + dpp_mov_d<CTRL>(send);
  }
}

// Sums over the 16 lanes of each row of C values per lane (C in 1, 2, 4, 8).
// Returns, in physical lane l16, the total of value index l16 >> (4 - log2 C).
template <int C>
__device__ __forceinline__ double score_rowsum(double (&v)[C], int l16) {
  static_assert(C == 1 || C == 2 || C == 4 || C == 8, "1, 2, 4 or 8 sums per lane");
  if constexpr (C == 8) {
    score_halve<8, 0x128>(v, l16 & 8);
    score_halve<4, 0x141>(v, l16 & 4);
    score_halve<2, 0x4E>(v, l16 & 2);
    return v[0] + dpp_mov_d<0xB1>(v[0]);
  } else if constexpr (C == 4) {
    score_halve<4, 0x128>(v, l16 & 8);
    score_halve<2, 0x141>(v, l16 & 4);
    double r = v[0] + dpp_mov_d<0x4E>(v[0]);
    return r + dpp_mov_d<0xB1>(r);
  } else if constexpr (C == 2) {
    score_halve<2, 0x128>(v, l16 & 8);
    double r = v[0] + dpp_mov_d<0x141>(v[0]);
    r = r + dpp_mov_d<0x4E>(r);
    return r + dpp_mov_d<0xB1>(r);
  } else {
    double r = v[0] + dpp_mov_d<0x128>(v[0]);
    r = r + dpp_mov_d<0x141>(r);
    r = r + dpp_mov_d<0x4E>(r);
    return r + dpp_mov_d<0xB1>(r);
  }
}

// P = 64-dim passes (D <= 64 * P), STEPS = 4-block wave steps per wave,
// GT = query heads per LDS stage.  FULL: D % 64 == 0 and q, lo, hi 16-byte
// aligned (whole passes, vector loads); otherwise dims past D are zeroed
// element by element.  PG: paged, batched bounds (lo/hi are pages [P, D],
// a.n is the block table's row width, a row's blocks past its request's
// count are not scored, and a block on an invalid page gets key 0).
// WV: waves per workgroup (a chunk is WV * 4 * STEPS blocks).  SIG (the
// one-launch step): the keys are stored agent-coherent and, once all of the
// workgroup's stores have completed, the chunk's flag of every query head of
// the group is set; the query values are requested before the bounds (one
// stage: G <= GT and GT * 64 * P <= blockDim).
template <typename Q, int P, int STEPS, bool FULL, int GT, bool PG = false, bool SIG = false,
          int WV = kScoreWaves>
__device__ __forceinline__ void score_wg(const ScoreArgs& a, int wg,
                                         const Paging& pg = Paging{}) {
  constexpr int C = GT * STEPS;           // (head, block) sums per wave
  constexpr int QN = GT * 64 * P;         // staged query values
  __shared__ __align__(16) double s_q[QN];
  __shared__ __align__(16) uint32_t s_m[QN];
  __shared__ uint32_t s_rng[SIG ? WV : 1][GT][2];   // SIG: per wave and head, key range
  const int G = a.hq / a.hkv;
  const int kv = wg / a.chunks;
  const int chunk = wg % a.chunks;
  const int h0 = kv * G;
  const int lane = lane_id();
  const int l16 = lane & 15;
  const int c = score_lane(l16);              // logical lane
  const int sub = lane >> 4;                  // block within a 4-block step
  const int wave_base = (chunk * WV + wave_id()) * (4 * STEPS);
  // PG: the table entries and the row's block count are requested together
  // (the entries' loads are bounded by the table width, not by the count)
  int pgs[PG ? STEPS : 1];
  if constexpr (PG) {
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int nb = wave_base + 4 * s + sub;
      pgs[s] = pg_bounds_row(pg, kv, a.n, nb, nb < a.n);
    }
  }
  const int nv = PG ? pg_blocks(pg, kv, a.n) : a.n;   // blocks of this row
  if (PG && chunk * WV * 4 * STEPS >= nv) return;   // whole workgroup
  const Q* qbase = reinterpret_cast<const Q*>(a.q) + (size_t)h0 * a.d;
  // SIG: this thread's query value goes out before the bounds, so the
  // staging below does not wait behind their round trip
  float qpre = 0.f;
  if constexpr (SIG) {
    const int x = threadIdx.x;
    const int gi = x / (64 * P), dim = x % (64 * P);
    const bool ok = x < QN && gi < G && dim < a.d;
    const Q qr = qbase[ok ? (size_t)gi * a.d + dim : 0];
    qpre = ok ? cvt(qr) : 0.f;
    __builtin_amdgcn_sched_barrier(0);
  }
  auto stage_q = [&] {
    if ((int)threadIdx.x < QN) {
      s_q[threadIdx.x] = (double)qpre;
      s_m[threadIdx.x] = qpre >= 0.f ? 0u : ~0u;   // lo where q < 0 or q is NaN
    }
    __syncthreads();
  };
  // every lo/hi load of the wave is issued before any arithmetic, with no
  // branch around a load: blocks past n read row 0 and are not stored
  float4 lv[STEPS][P], hv[STEPS][P];
  int dead = 0;   // PG: bit s set when this lane's block of step s has no page
  size_t rows[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int nb = wave_base + 4 * s + sub;
    const bool valid = nb < nv;
    if constexpr (PG) {
      const int page = valid ? pgs[s] : -1;
      dead |= (page < 0) << s;
      rows[s] = page >= 0 ? (size_t)page : 0;
    } else {
      rows[s] = (size_t)kv * a.n + (valid ? nb : 0);
    }
  }
  bool b16 = false;
  if constexpr (sizeof(Q) == 2) b16 = a.lb != 0;
  if constexpr (sizeof(Q) == 2) if (b16) {
    // 16-bit bounds: a lane's four dims are 8 bytes; the raw words are kept
    // in .x / .y and widened below, once every load is in flight
    const uint16_t* lb16 = static_cast<const uint16_t*>(a.lo);
    const uint16_t* hb16 = static_cast<const uint16_t*>(a.hi);
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const uint16_t* lrow = lb16 + rows[s] * a.d;
      const uint16_t* hrow = hb16 + rows[s] * a.d;
#pragma unroll
      for (int j = 0; j < P; ++j) {
        const int d0 = 64 * j + 4 * c;
        uint2 l2, h2;
        if constexpr (FULL) {
          const int dd = 64 * j < a.d ? d0 : 0;   // passes past D: unused
          l2 = *reinterpret_cast<const uint2*>(lrow + dd);
          h2 = *reinterpret_cast<const uint2*>(hrow + dd);
        } else {
          uint32_t l4[4], h4[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const bool ok = d0 + t < a.d;
            l4[t] = ld_or(lrow, (int64_t)(d0 + t), ok, (uint16_t)0);
            h4[t] = ld_or(hrow, (int64_t)(d0 + t), ok, (uint16_t)0);
          }
          l2 = make_uint2(l4[0] | (l4[1] << 16), l4[2] | (l4[3] << 16));
          h2 = make_uint2(h4[0] | (h4[1] << 16), h4[2] | (h4[3] << 16));
        }
        lv[s][j] = make_float4(__uint_as_float(l2.x), __uint_as_float(l2.y), 0.f, 0.f);
        hv[s][j] = make_float4(__uint_as_float(h2.x), __uint_as_float(h2.y), 0.f, 0.f);
      }
    }
    if constexpr (SIG) stage_q();   // while the bounds travel
#pragma unroll
    for (int s = 0; s < STEPS; ++s)
#pragma unroll
      for (int j = 0; j < P; ++j) {
        float f[4];
        Unpack<Q>::run(__float_as_uint(lv[s][j].x), f);
        Unpack<Q>::run(__float_as_uint(lv[s][j].y), f + 2);
        lv[s][j] = make_float4(f[0], f[1], f[2], f[3]);
        Unpack<Q>::run(__float_as_uint(hv[s][j].x), f);
        Unpack<Q>::run(__float_as_uint(hv[s][j].y), f + 2);
        hv[s][j] = make_float4(f[0], f[1], f[2], f[3]);
      }
  }
  if (!b16) {
    const float* lb32 = static_cast<const float*>(a.lo);
    const float* hb32 = static_cast<const float*>(a.hi);
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const float* lrow = lb32 + rows[s] * a.d;
      const float* hrow = hb32 + rows[s] * a.d;
#pragma unroll
      for (int j = 0; j < P; ++j) {
        const int d0 = 64 * j + 4 * c;
        if constexpr (FULL) {
          const int dd = 64 * j < a.d ? d0 : 0;   // passes past D: unused
          lv[s][j] = *reinterpret_cast<const float4*>(lrow + dd);
          hv[s][j] = *reinterpret_cast<const float4*>(hrow + dd);
        } else {
          float l4[4], h4[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const bool ok = d0 + t < a.d;
            l4[t] = ld_or(lrow, (int64_t)(d0 + t), ok, 0.f);
            h4[t] = ld_or(hrow, (int64_t)(d0 + t), ok, 0.f);
          }
          lv[s][j] = make_float4(l4[0], l4[1], l4[2], l4[3]);
          hv[s][j] = make_float4(h4[0], h4[1], h4[2], h4[3]);
        }
      }
    }
    if constexpr (SIG) stage_q();
  }
  for (int gb = 0; gb < G; gb += GT) {
    if constexpr (!SIG) {   // SIG: staged once, above
      if (gb) __syncthreads();   // previous stage fully read
      for (int x = threadIdx.x; x < QN; x += blockDim.x) {
        const int gi = x / (64 * P), dim = x % (64 * P);
        const bool ok = gb + gi < G && dim < a.d;
        const float qv = ok ? cvt(qbase[(size_t)(gb + gi) * a.d + dim]) : 0.f;
        s_q[x] = (double)qv;
        s_m[x] = qv >= 0.f ? 0u : ~0u;   // lo where q < 0 or q is NaN
      }
      __syncthreads();
    }
    double acc[C];
#pragma unroll
    for (int i = 0; i < C; ++i) acc[i] = 0.0;
#pragma unroll
    for (int gi = 0; gi < GT; ++gi) {
#pragma unroll
      for (int j = 0; j < P; ++j) {
        if (FULL && 64 * j >= a.d) continue;
        const int x = gi * 64 * P + 64 * j + 4 * c;
        const double2 q01 = *reinterpret_cast<const double2*>(s_q + x);
        const double2 q23 = *reinterpret_cast<const double2*>(s_q + x + 2);
        const uint4 mk = *reinterpret_cast<const uint4*>(s_m + x);
        const double qd[4] = {q01.x, q01.y, q23.x, q23.y};
        const uint32_t mm[4] = {mk.x, mk.y, mk.z, mk.w};
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
          const float lvv[4] = {lv[s][j].x, lv[s][j].y, lv[s][j].z, lv[s][j].w};
          const float hvv[4] = {hv[s][j].x, hv[s][j].y, hv[s][j].z, hv[s][j].w};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const uint32_t bits = (__float_as_uint(lvv[t]) & mm[t]) |
                                  (__float_as_uint(hvv[t]) & ~mm[t]);
            // exact product, one rounding; a zero q (dims past D) with a zero
            // bound adds +0.0, which leaves the sum unchanged
            acc[gi * STEPS + s] = fma(qd[t], (double)__uint_as_float(bits), acc[gi * STEPS + s]);
          }
        }
      }
    }
    double r = score_rowsum<C>(acc, l16);
    constexpr int LOGC = C == 8 ? 3 : (C == 4 ? 2 : (C == 2 ? 1 : 0));
    const int combo = l16 >> (4 - LOGC);
    const int gi = combo / STEPS, s = combo % STEPS;
    const int nb = wave_base + 4 * s + sub;
    const bool mine = (l16 & ((16 >> LOGC) - 1)) == 0 && nb < nv && gb + gi < G;
    if (r == 0.0) r = 0.0;
    const uint64_t key = (PG && ((dead >> s) & 1)) ? 0ull : score_key(r);
    if (mine) {
      const size_t o = (size_t)(h0 + gb + gi) * a.n + nb;
      if (a.scores) a.scores[o] = (float)r;
      if constexpr (SIG) st_agent(a.keys + o, key);
      else if (a.keys) a.keys[o] = key;
    }
    if constexpr (SIG) {
      // while the keys' stores travel: this wave's range of the high words
      // of its non-NaN keys, per query head (G <= GT: one stage)
      const uint32_t hw = (uint32_t)(key >> 32);
      const bool live = mine && key != 0ull;
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        const uint32_t mx = wave_ext_u32<true>(live && gi == g ? hw : 0u);
        const uint32_t mn = wave_ext_u32<false>(live && gi == g ? hw : 0xffffffffu);
        if (lane_id() == 0) {
          s_rng[wave_id()][g][0] = mx;
          s_rng[wave_id()][g][1] = mn;
        }
      }
    }
  }
  if constexpr (SIG) {
    // publish the chunk to every query head of the group
    wait_stores();
    __syncthreads();
    if (!a.drop && (int)threadIdx.x < G) {
      // The flag carries the chunk's range of key high words rounded
      // outward to 16 bits, (max >> 16) << 16 | (min >> 16), so that the
      // tail's top-K starts from the row's range without computing it.  It
      // is never 0: a non-NaN key's high word is at least 0x000FFFFF, and a
      // chunk without one gives 0x0000FFFF.
      uint32_t mx = 0u, mn = 0xffffffffu;
#pragma unroll
      for (int w = 0; w < WV; ++w) {
        mx = s_rng[w][threadIdx.x][0] > mx ? s_rng[w][threadIdx.x][0] : mx;
        mn = s_rng[w][threadIdx.x][1] < mn ? s_rng[w][threadIdx.x][1] : mn;
      }
      st_agent(a.sflag + (size_t)(h0 + threadIdx.x) * a.fstride + chunk,
               ((mx >> 16) << 16) | (mn >> 16));
    }
  }
}

}  // namespace stk
