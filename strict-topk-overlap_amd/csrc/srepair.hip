// The drop-in signed repair (strict_topk/signed_fused.py:148-193) for saved
// and hybrid predictions in one launch: one workgroup of 512 threads per
// query head does the job schedule, the signed block corrections and the
// guarded merge with the inline strict fallback.
//
// Reference:
//   strict_topk/signed_repair.py:18-82   _schedule (misses in selected-slot
//                                        order, then the wrong low blocks
//                                        in predicted-slot order; the kept
//                                        states; the max_extra_mass skip)
//   strict_topk/signed_fused.py:30-67    _corrections (each job's block-local
//                                        state; a hybrid negative rescaled by
//                                        exp(block_m - low_m))
//   strict_topk/signed_fused.py:70-145   _finalize (guards, merge, strict
//                                        fallback over the selected slots)
//
// A wrong low block is a predicted block, and the hybrid prediction holds
// the block-local state of every predicted block (strict_topk/kernels.py:
// 450-477 keeps all partials), computed from the same q, K, V with the same
// block-local arithmetic that _corrections repeats; the negative corrections
// are therefore taken from the prediction's state rows, and only the missed
// blocks' K/V tiles are read.  The three-launch form (k_schedule, k_jobs,
// k_finalize in signed.hip) re-reads every job's tile and chains three
// single-workgroup phases through global memory; here the head's whole input
// is requested at entry and every later phase works from registers and LDS:
//   1. selected and predicted rows, prediction scalars, query, low group and
//      every prediction state row (held in registers, RPT rows of four
//      columns per thread);
//   2. membership through two LDS byte maps over block IDs (IDs outside the
//      maps' range compare against the staged rows directly, so equality is
//      the reference's for any ID), and one packed scan that ranks the
//      misses and the candidate wrong blocks and counts the low hits;
//   3. every wave forms the kept maximum and the extra-mass test from the
//      staged slots by itself (no barrier); the waves issue their misses'
//      tile loads (wave w takes misses w, w + 8, ..., two in flight), sum the
//      kept states and the wrong blocks' corrections from the registered
//      rows while the tiles travel, then fold the misses into an online
//      softmax state;
//   4. one merge by D threads, the guard flags OR-ed through LDS, and on a
//      flagged head the strict softmax over the selected slots' tiles.
// Results agree with the three-launch form up to FP32 reduction order.
#include "srepair.hpp"
#include "step.hpp"
#include "tail.hpp"

#include <type_traits>

namespace stk {

constexpr int kSrMap = 8192;   // block IDs covered by the byte maps

template <typename T, int NCH, int UP, bool ONE, int RPT>
__global__ __launch_bounds__(kTailThreads) void k_srepair(SRepairArgs a) {
  using TT = TokTileW<T, NCH, UP>;
  constexpr int D = TT::D;
  constexpr int TPR = D / 4;                 // threads per state row
  constexpr int RG = kTailThreads / TPR;     // rows per pass of the state prefetch
  constexpr bool DB = ONE && RPT == 4 && UP * TT::QW + 4 * TT::NV <= 64;
  static_assert(kSrMap == 16 * kTailThreads, "one 16-byte clear per thread and map");
  static_assert(TPR <= STK_WAVE, "state rows wider than a wave");
  __shared__ __align__(16) uint8_t map_a[kSrMap], map_p[kSrMap];
  __shared__ int64_t s_a[kTailMaxK], s_p[kTailMaxK];
  __shared__ float s_pm[kTailMaxK], s_pl[kTailMaxK], s_mm[kTailMaxK], s_ml[kTailMaxK];
  __shared__ uint8_t s_hi[kTailMaxK], s_hit[kTailMaxK];
  __shared__ int jobs[kTailMaxK];
  __shared__ int s_scan[kTailWaves];
  __shared__ int s_bad;
  __shared__ float s_hl[kTailWaves], s_nl[kTailWaves], s_wm[kTailWaves], s_wl[kTailWaves];
  __shared__ __align__(16) float s_hu[kTailWaves][D];
  __shared__ __align__(16) float s_nu[kTailWaves][D];
  __shared__ __align__(16) float s_wu[kTailWaves][D];
  const int h = xcd_remap(blockIdx.x, gridDim.x), tid = threadIdx.x, w = wave_id();
  const int sa = a.sa, sp = a.sp, n = a.kv.n, b = a.kv.b;
  const int nmap = n < kSrMap ? n : kSrMap;
  const bool hybrid = a.hybrid != 0;
  const bool eps_on = hybrid && a.eps > 0.f;
  // ---- round trip 1: everything that does not depend on the schedule
  const int64_t aid = tid < sa ? load_id(a.a, a.atype, (int64_t)h * sa + tid) : -1;
  const int64_t pid = tid < sp ? load_id(a.p, a.ptype, (int64_t)h * sp + tid) : -1;
  const int64_t srow = (int64_t)h * sp + tid;
  const float pmv = ld_or(a.pm, srow, tid < sp, -INFINITY);
  const float plv = ld_or(a.pl, srow, tid < sp, 0.f);
  const uint8_t hv = hybrid && tid < sp ? a.high[srow] : (uint8_t)0;
  const float mmv = eps_on && tid < sp ? a.mass_m[srow] : -INFINITY;
  const float mlv = eps_on && tid < sp ? a.mass_l[srow] : 0.f;
  TT t;
  t.init();
  uint32_t qw[TT::QW];
  t.load_q(reinterpret_cast<const T*>(a.kv.q) + (size_t)h * D, qw);
  const int c4 = tid % TPR, rg = tid / TPR;
  float4 uu[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int r = rg + RG * j;
    const int64_t row = (int64_t)h * sp + (r < sp ? r : 0);
    uu[j] = *reinterpret_cast<const float4*>(a.pu + row * D + 4 * c4);
  }
  float lm = 0.f, ll = 0.f, luv = 0.f, lav = 0.f;
  if (hybrid) {
    lm = a.lm[h];
    ll = a.ll[h];
    if (tid < D) {
      luv = a.lu[(size_t)h * D + tid];
      lav = a.labs[(size_t)h * D + tid];
    }
  }
  reinterpret_cast<uint4*>(map_a)[tid] = make_uint4(0u, 0u, 0u, 0u);
  reinterpret_cast<uint4*>(map_p)[tid] = make_uint4(0u, 0u, 0u, 0u);
  if (tid < kTailMaxK) {
    s_a[tid] = aid;
    s_p[tid] = pid;
    s_pm[tid] = pmv;
    s_pl[tid] = plv;
    s_hi[tid] = hv;
    s_mm[tid] = mmv;
    s_ml[tid] = mlv;
  }
  if (tid == 0) s_bad = 0;
  __syncthreads();
  // ---- membership (signed_repair.py:27-30): P[p] in A, A[a] not in P
  const bool amap = tid < sa && aid >= 0 && aid < nmap;
  const bool pmap = tid < sp && pid >= 0 && pid < nmap;
  if (amap) map_a[aid] = 1;
  if (pmap) map_p[pid] = 1;
  __syncthreads();
  bool hit = false, miss = false;
  if (tid < sp) {
    if (pmap) {
      hit = map_a[pid] != 0;
    } else {
      for (int j = 0; j < sa; ++j) hit = hit || s_a[j] == pid;
    }
  }
  if (tid < sa) {
    bool in_p = false;
    if (amap) {
      in_p = map_p[aid] != 0;
    } else {
      for (int j = 0; j < sp; ++j) in_p = in_p || s_p[j] == aid;
    }
    miss = !in_p;
  }
  // candidate wrong blocks (predicted, not selected, low) and low hits
  const bool cw = hybrid && tid < sp && !hit && !hv;
  const bool lh = hybrid && tid < sp && hit && !hv;
  if (tid < kTailMaxK) s_hit[tid] = hit;
  int tot;
  const int pre = block_excl_scan1((int)miss | ((int)cw << 10) | ((int)lh << 20), s_scan, &tot);
  const int nmiss = tot & 1023, ncw = (tot >> 10) & 1023;
  const bool lowhit = hybrid && (tot >> 20) > 0;
  const int64_t qbase = (int64_t)h * a.cap;
  if (miss) {
    const int r = pre & 1023;
    jobs[r] = aid >= 0 && aid < n ? (int)aid : -1;
    store_id(a.queue, a.qtype, qbase + r, aid);
  }
  __syncthreads();
  // ---- kept maximum and the extra-mass test (signed_repair.py:58-72), the
  // same in every wave; lane l holds slots l, l + 64, ...
  float mk = -INFINITY;
  bool skip = false;
  float ex = 0.f;
  auto slots = [&](auto swn) {
    constexpr int SWN = decltype(swn)::value;
    bool keep[SWN], wrong[SWN];
#pragma unroll
    for (int c = 0; c < SWN; ++c) {
      const int p = c * STK_WAVE + lane_id();
      const bool ok = p < sp;
      const int pp = ok ? p : 0;
      keep[c] = ok && s_hit[pp] && (!hybrid || s_hi[pp]);
      wrong[c] = ok && lowhit && !s_hit[pp] && !s_hi[pp];
      mk = keep[c] ? fmaxf(mk, s_pm[pp]) : mk;
    }
    mk = wave_max_u(mk);
    if (eps_on && lowhit && ncw > 0) {
      const float ref = fmaxf(lm, mk);
      float dk = 0.f, dw = 0.f;
#pragma unroll
      for (int c = 0; c < SWN; ++c) {
        const int pp = keep[c] || wrong[c] ? c * STK_WAVE + lane_id() : 0;
        dk += keep[c] ? wexp(s_pm[pp], ref) * s_pl[pp] : 0.f;
        dw += wrong[c] ? wexp(s_mm[pp], ref) * s_ml[pp] : 0.f;
      }
      const float den = __expf(lm - ref) * ll + wave_sum_u(dk);
      ex = wave_sum_u(dw) / den;
      skip = ex <= a.eps;
    }
  };
  if (sp <= STK_WAVE) slots(std::integral_constant<int, 1>{});
  else slots(std::integral_constant<int, kTailMaxK / STK_WAVE>{});
  const bool subtract = lowhit && !skip;   // the wrong blocks are jobs
  if (cw && subtract) store_id(a.queue, a.qtype, qbase + nmiss + ((pre >> 10) & 1023), pid);
  // ---- round trip 2: the misses' tiles, wave w taking misses w, w + 8, ...
  const int kvh = h / (a.kv.hq / a.kv.hkv);
  const float scale = 1.0f / sqrtf((float)D);
  const T* K = reinterpret_cast<const T*>(a.kv.k);
  const T* V = reinterpret_cast<const T*>(a.kv.v);
  // an ID outside [0, n) has the empty state; its tile is read from block 0
  // and not used
  auto tile = [&](int x) {
    const int jb = jobs[x];
    return (((size_t)kvh * n + (jb >= 0 ? jb : 0)) * b) * D;
  };
  uint32_t kw[UP][TT::QW];
  uint4 vw[TT::NV];
  uint32_t kw2[UP][TT::QW];
  uint4 vw2[TT::NV];
  vm_drain();
  if (ONE && w < nmiss) t.load(K + tile(w), V + tile(w), 0, kw, vw);
  if (DB && w + kTailWaves < nmiss)
    t.load(K + tile(w + kTailWaves), V + tile(w + kTailWaves), 0, kw2, vw2);
  // ---- while they travel: the kept states relative to mk and the wrong
  // blocks' corrections in the low frame (block-local state times
  // exp(block_m - low_m)), from the registered rows
  float hl = 0.f, nl = 0.f;
  float4 hu = make_float4(0.f, 0.f, 0.f, 0.f), nu = hu;
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int r = rg + RG * j;
    const int rr = r < sp ? r : 0;
    const bool on = r < sp, ht = s_hit[rr], hh = s_hi[rr];
    const bool kp = on && ht && (!hybrid || hh);
    const bool wr = on && subtract && !ht && !hh;
    const float pm = s_pm[rr], pl = s_pl[rr];
    const float wk = kp ? wexp(pm, mk) : 0.f;
    const float wn = wr ? wexp(pm, lm) : 0.f;
    const float4 u4 = uu[j];
    hl += wk * pl;
    nl += wn * pl;
    hu.x += wk * u4.x; hu.y += wk * u4.y; hu.z += wk * u4.z; hu.w += wk * u4.w;
    nu.x += wn * u4.x; nu.y += wn * u4.y; nu.z += wn * u4.z; nu.w += wn * u4.w;
  }
#pragma unroll
  for (int off = TPR; off < STK_WAVE; off <<= 1) {
    hl += __shfl_xor(hl, off);
    nl += __shfl_xor(nl, off);
    hu.x += __shfl_xor(hu.x, off); hu.y += __shfl_xor(hu.y, off);
    hu.z += __shfl_xor(hu.z, off); hu.w += __shfl_xor(hu.w, off);
    nu.x += __shfl_xor(nu.x, off); nu.y += __shfl_xor(nu.y, off);
    nu.z += __shfl_xor(nu.z, off); nu.w += __shfl_xor(nu.w, off);
  }
  if (lane_id() < TPR) {
    *reinterpret_cast<float4*>(&s_hu[w][4 * c4]) = hu;
    *reinterpret_cast<float4*>(&s_nu[w][4 * c4]) = nu;
  }
  if (lane_id() == 0) {
    s_hl[w] = hl;
    s_nl[w] = nl;
  }
  // ---- the misses with the online softmax
  float m = -INFINITY, l = 0.f, acc[TT::ACC];
#pragma unroll
  for (int e = 0; e < TT::ACC; ++e) acc[e] = 0.f;
  auto job1 = [&](int x, const uint32_t (&kx)[UP][TT::QW], const uint4 (&vx)[TT::NV]) {
    if (jobs[x] >= 0) t.update(qw, kx, vx, 0, b, scale, m, l, acc);
  };
  if constexpr (DB) {
    for (int x = w; x < nmiss; x += 2 * kTailWaves) {
      job1(x, kw, vw);
      if (x + 2 * kTailWaves < nmiss)
        t.load(K + tile(x + 2 * kTailWaves), V + tile(x + 2 * kTailWaves), 0, kw, vw);
      if (x + kTailWaves < nmiss) {
        job1(x + kTailWaves, kw2, vw2);
        if (x + 3 * kTailWaves < nmiss)
          t.load(K + tile(x + 3 * kTailWaves), V + tile(x + 3 * kTailWaves), 0, kw2, vw2);
      }
    }
  } else if constexpr (ONE) {
    for (int x = w; x < nmiss; x += kTailWaves) {
      if (x != w) t.load(K + tile(x), V + tile(x), 0, kw, vw);
      job1(x, kw, vw);
    }
  } else {
    for (int x = w; x < nmiss; x += kTailWaves) {
      if (jobs[x] < 0) continue;
      for (int t0 = 0; t0 < b; t0 += TT::CH) {
        t.load(K + tile(x), V + tile(x), t0, kw, vw);
        t.update(qw, kw, vw, t0, b, scale, m, l, acc);
      }
    }
  }
  if (lane_id() == 0) {
    s_wm[w] = m;
    s_wl[w] = l;
  }
  t.store(s_wu[w], acc);
  __syncthreads();
  // ---- guarded merge (signed_fused.py:88-122), one thread per dim
  float frac = 1.f, o = 0.f;
  if (tid < D) {
    bool bad = false;
    float low_m = -INFINITY, low_l = 0.f, low_u = 0.f;
    if (lowhit) {
      float rl = 0.f, ru = 0.f;
#pragma unroll
      for (int g = 0; g < kTailWaves; ++g) {
        rl += s_nl[g];
        ru += s_nu[g][tid];
      }
      low_m = lm;
      low_l = ll - rl;
      low_u = luv - ru;
      frac = low_l / ll;
      const float cs = lav + fabsf(ru);
      bad = frac < a.min_remain || frac != frac || (fabsf(low_u) < a.cancel * cs && cs > 0.f);
    }
    float M = fmaxf(mk, low_m);
#pragma unroll
    for (int g = 0; g < kTailWaves; ++g) M = fmaxf(M, s_wm[g]);
    const float fk = wexp(mk, M), fl = wexp(low_m, M);
    float hls = 0.f, hus = 0.f;
#pragma unroll
    for (int g = 0; g < kTailWaves; ++g) {
      hls += s_hl[g];
      hus += s_hu[g][tid];
    }
    float den = fk * hls + fl * low_l;
    float num = fk * hus + fl * low_u;
#pragma unroll
    for (int g = 0; g < kTailWaves; ++g) {
      const float f = wexp(s_wm[g], M);
      den += f * s_wl[g];
      num += f * s_wu[g][tid];
    }
    o = num / den;
    if (hybrid) bad = bad || is_bad(o) || den <= 0.f || isinf(den);
    if (bad) s_bad = 1;
  }
  __syncthreads();
  const bool fallback = s_bad != 0;
  if (tid == 0) {
    a.bad[h] = fallback ? 1 : 0;
    a.remain[h] = frac;
    a.pos[h] = nmiss;
    a.total[h] = nmiss + (subtract ? ncw : 0);
    if (a.eps > 0.f) {
      a.approx[h] = (!fallback && skip) ? 1 : 0;
      a.extra[h] = (!fallback && skip) ? ex : 0.f;
    }
  }
  if (!fallback) {
    if (tid < D) a.out[(size_t)h * D + tid] = o;
    return;
  }
  // ---- strict fallback (signed_fused.py:123-142): the softmax over the
  // selected slots' tiles, wave w taking slots w, w + 8, ...
  float fm = -INFINITY, fz = 0.f, facc[TT::ACC];
#pragma unroll
  for (int e = 0; e < TT::ACC; ++e) facc[e] = 0.f;
  for (int x = w; x < sa; x += kTailWaves) {
    const int64_t id = s_a[x];
    if (id < 0 || id >= n) continue;
    const size_t off = (((size_t)kvh * n + (size_t)id) * b) * D;
    for (int t0 = 0; t0 < b; t0 += TT::CH) {
      t.load(K + off, V + off, t0, kw, vw);
      t.update(qw, kw, vw, t0, b, scale, fm, fz, facc);
    }
  }
  if (lane_id() == 0) {
    s_wm[w] = fm;
    s_wl[w] = fz;
  }
  t.store(s_wu[w], facc);
  __syncthreads();
  if (tid < D) {
    float M = -INFINITY;
#pragma unroll
    for (int g = 0; g < kTailWaves; ++g) M = fmaxf(M, s_wm[g]);
    float den = 0.f, num = 0.f;
#pragma unroll
    for (int g = 0; g < kTailWaves; ++g) {
      const float f = wexp(s_wm[g], M);
      den += f * s_wl[g];
      num += f * s_wu[g][tid];
    }
    a.out[(size_t)h * D + tid] = num / den;
  }
}

bool srepair_covers(int dtype, int b, int d, int sa, int sp, uintptr_t align) {
  if (dtype != DT_BF16 && dtype != DT_F16) return false;
  if (!tok_nch(dtype, d, b, align)) return false;
  if (sa < 1 || sp < 1 || sa > kTailMaxK || sp > kTailMaxK) return false;
  const int per_pass = kTailThreads * 4 / d;
  return (sp + per_pass - 1) / per_pass <= 16;
}

namespace {

template <typename T, int NCH, int UP, bool ONE>
int srepair_one(const SRepairArgs& a, int rpt, hipStream_t st) {
  const dim3 grid(a.kv.hq), block(kTailThreads);
  if (rpt == 4)
    hipLaunchKernelGGL((k_srepair<T, NCH, UP, ONE, 4>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((k_srepair<T, NCH, UP, ONE, 16>), grid, block, 0, st, a);
  return stk_check_launch("k_srepair");
}

}  // namespace

int launch_srepair(int dtype, const SRepairArgs& a, hipStream_t st) {
  const int b = a.kv.b, d = a.kv.d;
  const int nch = tok_nch(dtype, d, b, 0);
  const int up = tok_up(b);
  const bool one = b == 16 * up;
  const int per_pass = kTailThreads * 4 / d;
  const int rpt = (a.sp + per_pass - 1) / per_pass <= 4 ? 4 : 16;
  STK_DISPATCH_STEP(dtype, nch, {
    return up == 1 ? (one ? srepair_one<T, NCH, 1, true>(a, rpt, st)
                          : srepair_one<T, NCH, 1, false>(a, rpt, st))
                   : (one ? srepair_one<T, NCH, 2, true>(a, rpt, st)
                          : srepair_one<T, NCH, 2, false>(a, rpt, st));
  });
  return STK_EINVAL;
}

}  // namespace stk
