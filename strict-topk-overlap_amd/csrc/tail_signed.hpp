// Tail of the fused signed decode step: exact top-K of one query head's keys,
// then the hybrid grouping of its predicted states, the signed add/erase
// corrections and the guarded merge with the strict fallback, in one
// workgroup per head.
//
// Reference:
//   strict_topk/gqa.py:145-161           select_blocks (the keys' top-K)
//   strict_topk/kernels.py:94-117        _group (hybrid: high = mass >= tau *
//                                        total, low aggregate (m, l, u) and the
//                                        absolute envelope)
//   strict_topk/signed_repair.py:18-82   _schedule (misses, wrong low blocks,
//                                        kept states, the max_extra_mass skip)
//   strict_topk/signed_fused.py:30-67    _corrections (signed block states;
//                                        hybrid negatives in the low frame)
//   strict_topk/signed_fused.py:70-145   _finalize (guards, merge, fallback)
// The arithmetic is that of stk_speculate (hybrid) + stk_repair_signed with
// the fused rule; results agree up to FP32 reduction order.
//
// Layout (512 threads, every memory round trip issued as early as its
// inputs allow):
//   1. keys, predicted row, query row and every predicted state (m, l, u);
//      the u rows stay in registers (RPT rows of four columns per thread);
//   2. top-K (value bins, topk_bins.hpp) and one packed scan that ranks the
//      selected IDs and lists the misses; every wave issues the tile loads
//      of its misses at once (wave w takes misses w, w + 8, ..., two tiles
//      in flight), and wave 0 does the per-slot work (grouping, membership,
//      keep / low / wrong sets, the extra-mass test) while they travel;
//   3. the partial sums of the registered u rows: the kept states, the low
//      aggregate with its envelope, and the wrong low blocks' corrections.
//      A wrong block's correction in the reference (_corrections :52-61) is
//      its block-local state (max m, l, u of the recomputed tile) times
//      exp(m - low_m); that state is the prediction state this step's front
//      computed for the same block with the same arithmetic, so it is taken
//      from the registered rows instead of re-reading the tile; then the
//      missed tiles, folded with an online softmax;
//   4. one merge by D threads, the guard flags OR-ed through LDS, and on a
//      flagged head the strict softmax over the selected blocks, merged
//      from their exact block states (hits from the registered rows, misses
//      from the waves' online states).
#pragma once

#include <type_traits>

#include "topk_bins.hpp"
#include "tile2.hpp"
#include "tail.hpp"

namespace stk {

struct STailArgs {
  KV kv;                                  // q, k, v, hq, hkv, n, b, d
  const uint64_t* keys;                   // [hq, n]
  int k;                                  // selected per head
  int32_t* ids;                           // [hq, k] out, ascending
  const int32_t* p; int sp;               // predicted [hq, sp]
  const float* pm; const float* pl; const float* pu;   // predicted states
  int hybrid;                             // 1: hybrid prediction, 0: saved
  float tau, min_remaining, cancel_tol, eps;
  float* out;                             // [hq, d]
  uint8_t* bad; float* remain;            // [hq]
  uint8_t* approx; float* extra;          // [hq] or null when eps == 0
  int32_t* pos; int32_t* total;           // [hq] job counts
  Paging pg;                              // PG: paged, batched KV
};

// PG: paged, batched KV, as in tail_head (min(k, n) selected of the
// request's n blocks; pages loaded with the keys).
template <typename T, int NCH, int UP, bool ONE, int KPT, int RPT, bool PG = false>
__device__ __forceinline__ void stail_head(const STailArgs& a) {
  using TT = TokTileW<T, NCH, UP>;
  constexpr int D = TT::D;
  constexpr int TPR = D / 4;              // threads per state row (16-byte loads)
  constexpr int RG = kTailThreads / TPR;  // rows per pass of the state prefetch
  constexpr int SW = kTailMaxK / STK_WAVE;   // slot words of wave 0
  // two tile buffers in flight when they fit the register budget
  constexpr bool DB = ONE && RPT == 4 && UP * TT::QW + 4 * TT::NV <= 64;
  __shared__ int map[kTailMapN];
  __shared__ int sel[kTailMaxK], miss[kTailMaxK], pids[kTailMaxK];
  __shared__ float s_pm[kTailMaxK], s_pl[kTailMaxK];
  __shared__ TopkBinsLds tb;
  __shared__ int s_scan[kTailWaves];
  __shared__ int s_nw, s_lowhit, s_skip, s_bad;
  __shared__ float s_lowm, s_ll, s_mk, s_mu, s_extra;
  __shared__ uint64_t s_keep[SW], s_low[SW], s_wrong[SW], s_used[SW];
  // partial sums of the registered rows, one row per wave (row groups that
  // share a wave are folded in registers first)
  __shared__ float s_hl[kTailWaves], s_nl[kTailWaves], s_sl[kTailWaves];
  __shared__ __align__(16) float s_hu[kTailWaves][D];
  __shared__ __align__(16) float s_lu[kTailWaves][D];
  __shared__ __align__(16) float s_la[kTailWaves][D];
  __shared__ __align__(16) float s_nu[kTailWaves][D];
  __shared__ __align__(16) float s_su[kTailWaves][D];
  __shared__ float s_wm[kTailWaves], s_wl[kTailWaves];
  __shared__ float s_wu[kTailWaves][D];
  __shared__ int mtk[PG ? kTailMaxK : 1];   // PG: tokens of each listed miss
  const int h = xcd_remap(blockIdx.x, gridDim.x);   // a KV group's heads on one XCD
  const int nrow = a.kv.n, sp = a.sp;
  const int tid = threadIdx.x, w = wave_id();
  const int G = a.kv.hq / a.kv.hkv;
  const bool hybrid = a.hybrid != 0;
  // ---- round trip 1: every load that does not depend on the top-K
  uint64_t key[KPT];
  topk_load<KPT>(a.keys + (size_t)h * nrow, nrow, key);
  // PG: the pages of this thread's blocks and the row's block count come
  // with the keys (the dense step computes its KV head later, off the path
  // of the entry loads)
  const int kvp = PG ? h / G : 0;
  int pgk[PG ? KPT : 1];
  if constexpr (PG) {
#pragma unroll
    for (int i = 0; i < KPT; ++i)
      pgk[i] = pg_page(a.pg, kvp, nrow, tid * KPT + i, tid * KPT + i < nrow);
  }
  const int n = PG ? pg_blocks(a.pg, kvp, nrow) : nrow;   // blocks of the row
  const int rtok = PG ? pg_row_tokens(a.pg, kvp) : 0;     // PG: tokens of the request
  const int kk = PG ? (a.k < n ? a.k : n) : a.k;           // selected
  const int pid = (int)ld_or(a.p, (int64_t)h * sp + tid, tid < sp, (int32_t)-1);
  TT t;
  t.init();
  uint32_t qw[TT::QW];
  t.load_q(reinterpret_cast<const T*>(a.kv.q) + (size_t)h * D, qw);
  const float pmv = ld_or(a.pm, (int64_t)h * sp + tid, tid < sp, -INFINITY);
  const float plv = ld_or(a.pl, (int64_t)h * sp + tid, tid < sp, 0.f);
  const int c4 = tid % TPR, rg = tid / TPR;
  float4 uu[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int r = rg + RG * j;
    const int64_t row = (int64_t)h * sp + (r < sp ? r : 0);
    uu[j] = *reinterpret_cast<const float4*>(a.pu + row * D + 4 * c4);
  }
  // ---- membership map (max predicted slot + 1 per block ID), cleared here
  // and filled between the top-K's first two barriers
  for (int i = tid; i < n; i += kTailThreads) map[i] = 0;
  // every slot entry is written (empty past sp): the row sums below read
  // entries past sp with zero weight, and LDS holds whatever an earlier
  // workgroup left there (NaN patterns included, and 0 * NaN is NaN)
  if (tid < kTailMaxK) {
    pids[tid] = pid;
    s_pm[tid] = pmv;
    s_pl[tid] = plv;
  }
  if (tid == 0) s_bad = 0;
  auto fill_map = [&] {
    if (tid < sp && pid >= 0 && pid < n) atomicMax(&map[pid], tid + 1);
  };
  // ---- exact top-K: a bit per selected key of this thread
  uint32_t flags = 0;
  if (!PG || kk > 0) {
    flags = topk_bins_flags<KPT>(key, n, kk, tb, fill_map);
  } else {
    __syncthreads();
    fill_map();
  }
  // ---- ranks: selected IDs in ascending block order, and the misses
  // (selected, not predicted) among them in the same order, from one scan
  // of packed counts (PG: a miss on an invalid page or with no tokens has
  // the empty state and is not listed; the list holds the misses' pages
  // instead of their IDs, and their token counts beside them)
  uint32_t mflags = 0;
  int mtok[PG ? KPT : 1];
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int idx = tid * KPT + i;
    const bool on = (flags >> i) & 1u;
    const int mv = map[on ? idx : 0];
    bool ms = on && mv == 0;
    if constexpr (PG) {
      mtok[i] = pg_block_tokens(rtok, idx, a.kv.b);
      ms = ms && pgk[i] >= 0 && mtok[i] > 0;
    }
    mflags |= (uint32_t)ms << i;
  }
  int total;
  const int pre = block_excl_scan1(__popc(flags) | (__popc(mflags) << 16), s_scan, &total);
  int spos = pre & 0xffff, mpos = pre >> 16;
  const int nm = total >> 16;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int idx = tid * KPT + i;
    if ((flags >> i) & 1u) {
      sel[spos++] = idx;
      map[idx] |= kSelFlag;   // this thread's block: no other writer
    }
    if ((mflags >> i) & 1u) {
      if constexpr (PG) {
        miss[mpos] = pgk[i];
        mtk[mpos] = mtok[i];
      } else {
        miss[mpos] = idx;
      }
      ++mpos;
    }
  }
  __syncthreads();
  // ---- per-slot work (wave 0), lane l holding slots l, l + 64, ...; SWN
  // slot words, one when SP <= 64 (a single wave runs this part alone, so
  // its instruction count is latency)
  auto slots = [&](auto swn) {
    constexpr int SWN = decltype(swn)::value;
    float pm_[SWN], pl_[SWN];
    bool ok[SWN], hit[SWN], real[SWN], used[SWN];
    float gm = -INFINITY, mu = -INFINITY;
#pragma unroll
    for (int c = 0; c < SWN; ++c) {
      const int p = c * STK_WAVE + lane_id();
      ok[c] = p < sp;
      pm_[c] = ok[c] ? s_pm[p] : -INFINITY;
      pl_[c] = ok[c] ? s_pl[p] : 0.f;
      const int id = ok[c] ? pids[p] : -1;
      real[c] = id >= 0 && id < n;
      const int mv = real[c] ? map[id] : 0;
      hit[c] = (mv & kSelFlag) != 0;
      // each selected block once (its highest slot), for the strict merge
      used[c] = hit[c] && (mv & ~kSelFlag) == p + 1;
      gm = fmaxf(gm, pm_[c]);
      mu = used[c] ? fmaxf(mu, pm_[c]) : mu;
    }
    mu = wave_max_u(mu);
    bool high[SWN], low[SWN], wrong[SWN], keep[SWN];
    float lowm = 0.f, ll = 0.f;
    bool lowhit = false;
    if (hybrid) {
      // kernels.py:102-117: mass under the predicted-set softmax
      gm = wave_max_u(gm);
      float tot = 0.f;
#pragma unroll
      for (int c = 0; c < SWN; ++c) tot += wexp(pm_[c], gm) * pl_[c];
      tot = wave_sum_u(tot);
      float lm = -INFINITY;
#pragma unroll
      for (int c = 0; c < SWN; ++c) {
        high[c] = ok[c] && wexp(pm_[c], gm) * pl_[c] >= a.tau * tot;
        low[c] = ok[c] && !high[c];
        lm = low[c] ? fmaxf(lm, pm_[c]) : lm;
      }
      lm = wave_max_u(lm);
      lowm = lm == -INFINITY ? 0.f : lm;
      float x = 0.f;
      bool lh = false;
#pragma unroll
      for (int c = 0; c < SWN; ++c) {
        x += low[c] ? wexp(pm_[c], lowm) * pl_[c] : 0.f;
        lh = lh || (hit[c] && low[c]);
      }
      ll = wave_sum_u(x);
      lowhit = __ballot(lh) != 0ull;
#pragma unroll
      for (int c = 0; c < SWN; ++c) {
        // an ID outside [0, n) has the empty state (-inf, 0, 0): nothing to
        // subtract, and no tile to read
        wrong[c] = lowhit && low[c] && !hit[c] && real[c];
        keep[c] = hit[c] && high[c];
      }
    } else {
#pragma unroll
      for (int c = 0; c < SWN; ++c) {
        high[c] = low[c] = wrong[c] = false;
        keep[c] = hit[c];
      }
    }
    float mk = -INFINITY;
#pragma unroll
    for (int c = 0; c < SWN; ++c) mk = keep[c] ? fmaxf(mk, pm_[c]) : mk;
    mk = wave_max_u(mk);
    // signed_repair.py:61-72: skip the wrong blocks when their mass is small
    bool skip = false;
    float ex = 0.f;
    bool anyw = false;
#pragma unroll
    for (int c = 0; c < SWN; ++c) anyw = anyw || wrong[c];
    if (hybrid && a.eps > 0.f && __ballot(anyw) != 0ull) {
      const float ref = fmaxf(lowm, mk);
      float dk = 0.f, dw = 0.f;
#pragma unroll
      for (int c = 0; c < SWN; ++c) {
        dk += keep[c] ? wexp(pm_[c], ref) * pl_[c] : 0.f;
        dw += wrong[c] ? wexp(pm_[c], ref) * pl_[c] : 0.f;
      }
      const float denom = wexp(lowm, ref) * ll + wave_sum_u(dk);
      ex = wave_sum_u(dw) / denom;
      skip = ex <= a.eps;
    }
    int nw = 0;
#pragma unroll
    for (int c = 0; c < SWN; ++c) {
      const uint64_t wb = __ballot(wrong[c] && !skip);
      nw += (int)__popcll(wb);
      const uint64_t kb = __ballot(keep[c]), lb = __ballot(low[c]), ub = __ballot(used[c]);
      if (lane_id() == 0) {
        s_keep[c] = kb;
        s_low[c] = lb;
        s_wrong[c] = wb;
        s_used[c] = ub;
      }
    }
    if (lane_id() == 0) {
      s_nw = nw;
      s_lowm = lowm;
      s_ll = ll;
      s_mk = mk;
      s_mu = mu;
      s_lowhit = lowhit ? 1 : 0;
      s_skip = skip ? 1 : 0;
      s_extra = skip ? ex : 0.f;
    }
#pragma unroll
    for (int c = SWN; c < SW; ++c)
      if (lane_id() == 0) s_keep[c] = s_low[c] = s_wrong[c] = s_used[c] = 0ull;
  };
  // ---- round trip 2: wave w streams misses w, w + 8, ..., two tiles in
  // flight when they fit
  const int kvh = PG ? kvp : h / G;
  const float scale = 1.0f / sqrtf((float)D);
  const T* K = reinterpret_cast<const T*>(a.kv.k);
  const T* V = reinterpret_cast<const T*>(a.kv.v);
  auto tile = [&](int x) {
    const size_t page = PG ? (size_t)miss[x] : (size_t)kvh * n + miss[x];
    return (page * a.kv.b) * D;
  };
  uint32_t kw[UP][TT::QW];
  uint4 vw[TT::NV];
  uint32_t kw2[UP][TT::QW];
  uint4 vw2[TT::NV];
  // the entry loads (u rows, query) returned during the top-K; after this
  // wait the compiler knows it, and the sums below never wait for the tiles
  vm_drain();
  if (ONE && w < nm) t.load(K + tile(w), V + tile(w), 0, kw, vw);
  if (DB && w + kTailWaves < nm)
    t.load(K + tile(w + kTailWaves), V + tile(w + kTailWaves), 0, kw2, vw2);
  // the selected IDs go out behind the tile loads
  for (int i = tid; i < a.k; i += kTailThreads)
    a.ids[(size_t)h * a.k + i] = (!PG || i < kk) ? sel[i] : -1;
  if (w == 0) {
    if (sp <= STK_WAVE) slots(std::integral_constant<int, 1>{});
    else slots(std::integral_constant<int, SW>{});
  }
  __syncthreads();
  const int nw = s_nw;
  const float lowm = s_lowm, mk = s_mk, mu = s_mu;
  // ---- partial sums of the registered u rows: kept states relative to mk;
  // the low aggregate, its envelope and the wrong blocks' corrections
  // relative to low_m
  float hl = 0.f, nl = 0.f, sl = 0.f;
  float4 hu = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 lu = hu, la = hu, nu = hu, su = hu;
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int r = rg + RG * j;   // < 16 * RG <= 512
    const int rr = r < kTailMaxK ? r : 0;
    const int wd = rr >> 6, bit = rr & 63;
    // mask words straight from LDS (a private array indexed per thread
    // would live in scratch memory, whose loads share the vector memory
    // counter with the tile loads in flight and would wait for them)
    const uint64_t kword = s_keep[wd], lword = s_low[wd], wword = s_wrong[wd];
    const uint64_t uword = s_used[wd];
    const bool kp = r < sp && ((kword >> bit) & 1ull);
    const bool lo = r < sp && ((lword >> bit) & 1ull);
    const bool wr = r < sp && ((wword >> bit) & 1ull);
    const bool us = r < sp && ((uword >> bit) & 1ull);
    const float pm = s_pm[rr], pl = s_pl[rr];
    const float wk = kp ? wexp(pm, mk) : 0.f;
    const float wl = lo ? wexp(pm, lowm) : 0.f;
    const float wn = wr ? wl : 0.f;
    const float ws = us ? wexp(pm, mu) : 0.f;
    // rows past sp were loaded from row 0 (or a stand-in buffer): zero them
    const float4 u4 = r < sp ? uu[j] : make_float4(0.f, 0.f, 0.f, 0.f);
    hl += wk * pl;
    nl += wn * pl;
    sl += ws * pl;
    hu.x += wk * u4.x; hu.y += wk * u4.y; hu.z += wk * u4.z; hu.w += wk * u4.w;
    lu.x += wl * u4.x; lu.y += wl * u4.y; lu.z += wl * u4.z; lu.w += wl * u4.w;
    la.x += wl * fabsf(u4.x); la.y += wl * fabsf(u4.y);
    la.z += wl * fabsf(u4.z); la.w += wl * fabsf(u4.w);
    nu.x += wn * u4.x; nu.y += wn * u4.y; nu.z += wn * u4.z; nu.w += wn * u4.w;
    su.x += ws * u4.x; su.y += ws * u4.y; su.z += ws * u4.z; su.w += ws * u4.w;
  }
  // fold the row groups of this wave (lanes with the same columns)
#pragma unroll
  for (int off = TPR; off < STK_WAVE; off <<= 1) {
    hl += __shfl_xor(hl, off);
    nl += __shfl_xor(nl, off);
    hu.x += __shfl_xor(hu.x, off); hu.y += __shfl_xor(hu.y, off);
    hu.z += __shfl_xor(hu.z, off); hu.w += __shfl_xor(hu.w, off);
    lu.x += __shfl_xor(lu.x, off); lu.y += __shfl_xor(lu.y, off);
    lu.z += __shfl_xor(lu.z, off); lu.w += __shfl_xor(lu.w, off);
    la.x += __shfl_xor(la.x, off); la.y += __shfl_xor(la.y, off);
    la.z += __shfl_xor(la.z, off); la.w += __shfl_xor(la.w, off);
    nu.x += __shfl_xor(nu.x, off); nu.y += __shfl_xor(nu.y, off);
    nu.z += __shfl_xor(nu.z, off); nu.w += __shfl_xor(nu.w, off);
    sl += __shfl_xor(sl, off);
    su.x += __shfl_xor(su.x, off); su.y += __shfl_xor(su.y, off);
    su.z += __shfl_xor(su.z, off); su.w += __shfl_xor(su.w, off);
  }
  // a wave holds STK_WAVE / TPR row groups; with TPR > STK_WAVE (D = 512)
  // a row group spans waves, which the fused step does not support
  static_assert(TPR <= STK_WAVE, "state rows wider than a wave");
  if (lane_id() < TPR) {
    *reinterpret_cast<float4*>(&s_hu[w][4 * c4]) = hu;
    *reinterpret_cast<float4*>(&s_lu[w][4 * c4]) = lu;
    *reinterpret_cast<float4*>(&s_la[w][4 * c4]) = la;
    *reinterpret_cast<float4*>(&s_nu[w][4 * c4]) = nu;
    *reinterpret_cast<float4*>(&s_su[w][4 * c4]) = su;
  }
  if (lane_id() == 0) {
    s_hl[w] = hl;
    s_nl[w] = nl;
    s_sl[w] = sl;
  }
  // ---- the misses' states with the online softmax
  float m = -INFINITY, l = 0.f, acc[TT::ACC];
#pragma unroll
  for (int e = 0; e < TT::ACC; ++e) acc[e] = 0.f;
  // one whole-block tile of miss x (PG: a partly filled block weights only
  // its first mtk[x] tokens)
  auto upd1 = [&](int x, const uint32_t (&kx)[UP][TT::QW], const uint4 (&vx)[TT::NV]) {
    if (PG && mtk[x] < a.kv.b) t.template update<true>(qw, kx, vx, 0, mtk[x], scale, m, l, acc);
    else t.update(qw, kx, vx, 0, a.kv.b, scale, m, l, acc);
  };
  if constexpr (DB) {
    // two register buffers: tile x computes while tile x + 8 is in flight
    for (int x = w; x < nm; x += 2 * kTailWaves) {
      upd1(x, kw, vw);
      if (x + 2 * kTailWaves < nm)
        t.load(K + tile(x + 2 * kTailWaves), V + tile(x + 2 * kTailWaves), 0, kw, vw);
      if (x + kTailWaves < nm) {
        upd1(x + kTailWaves, kw2, vw2);
        if (x + 3 * kTailWaves < nm)
          t.load(K + tile(x + 3 * kTailWaves), V + tile(x + 3 * kTailWaves), 0, kw2, vw2);
      }
    }
  } else if constexpr (ONE) {
    for (int x = w; x < nm; x += kTailWaves) {
      if (x != w) t.load(K + tile(x), V + tile(x), 0, kw, vw);
      upd1(x, kw, vw);
    }
  } else {
    for (int x = w; x < nm; x += kTailWaves) {
      const int lim = PG ? mtk[x] : a.kv.b;
      for (int t0 = 0; t0 < lim; t0 += TT::CH) {
        t.load(K + tile(x), V + tile(x), t0, kw, vw);
        if (PG && t0 + TT::CH > lim) t.template update<true>(qw, kw, vw, t0, lim, scale, m, l, acc);
        else t.update(qw, kw, vw, t0, a.kv.b, scale, m, l, acc);
      }
    }
  }
  if (lane_id() == 0) {
    s_wm[w] = m;
    s_wl[w] = l;
  }
  t.store(s_wu[w], acc);
  __syncthreads();
  // ---- guarded merge (signed_fused.py:98-122), one thread per dim
  float frac = 1.f, o = 0.f;
  const bool lowhit = hybrid && s_lowhit != 0;
  if (tid < D) {
    float lm_eff = -INFINITY, lowl = 0.f, lowu = 0.f;
    bool bad = false;
    if (lowhit) {
      float nls = 0.f, nus = 0.f, lus = 0.f, env = 0.f;
#pragma unroll
      for (int g = 0; g < kTailWaves; ++g) {
        nls += s_nl[g];
        nus += s_nu[g][tid];
        lus += s_lu[g][tid];
        env += s_la[g][tid];
      }
      const float ll = s_ll;
      const float removed = -nus;
      lowl = ll - nls;
      lowu = lus + removed;
      frac = lowl / ll;
      const float cs = env + fabsf(removed);
      bad = (frac < a.min_remaining) || (frac != frac) ||
            (fabsf(lowu) < a.cancel_tol * cs && cs > 0.f);
      lm_eff = lowm;
    }
    float M = fmaxf(mk, lm_eff);
#pragma unroll
    for (int x = 0; x < kTailWaves; ++x) M = fmaxf(M, s_wm[x]);
    const float fk = wexp(mk, M), fl = wexp(lm_eff, M);
    float hls = 0.f, hus = 0.f;
#pragma unroll
    for (int g = 0; g < kTailWaves; ++g) {
      hls += s_hl[g];
      hus += s_hu[g][tid];
    }
    float den = fk * hls + fl * lowl;
    float num = fk * hus + fl * lowu;
#pragma unroll
    for (int x = 0; x < kTailWaves; ++x) {
      const float f = wexp(s_wm[x], M);
      den += f * s_wl[x];
      num += f * s_wu[x][tid];
    }
    o = num / den;
    if (hybrid)
      bad = bad || !isfinite(o) || den <= 0.f || isinf(den);
    if (bad) s_bad = 1;
  }
  __syncthreads();
  const bool fallback = s_bad != 0;
  if (tid == 0) {
    a.bad[h] = fallback ? 1 : 0;
    a.remain[h] = frac;
    a.pos[h] = nm;
    a.total[h] = nm + nw;
    if (a.approx) {
      a.approx[h] = (!fallback && s_skip) ? 1 : 0;
      a.extra[h] = fallback ? 0.f : s_extra;
    }
  }
  if (!fallback) {
    if (tid < D) a.out[(size_t)h * D + tid] = o;
    return;
  }
  // ---- strict fallback (signed_fused.py:123-142): the softmax over the
  // selected blocks alone.  Every selected block's exact block-local state
  // is at hand (the predicted ones in the registered rows, each block once;
  // the missed ones in the waves' online states), so the fallback merges
  // those with positive weights (no signed term, no second pass over the
  // tiles) instead of streaming the selected tiles again.
  if (tid < D) {
    float M = mu;
#pragma unroll
    for (int x = 0; x < kTailWaves; ++x) M = fmaxf(M, s_wm[x]);
    const float fs = wexp(mu, M);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int g = 0; g < kTailWaves; ++g) {
      den += s_sl[g];
      num += s_su[g][tid];
    }
    num *= fs;
    den *= fs;
#pragma unroll
    for (int x = 0; x < kTailWaves; ++x) {
      const float f = wexp(s_wm[x], M);
      den += f * s_wl[x];
      num += f * s_wu[x][tid];
    }
    a.out[(size_t)h * D + tid] = num / den;
  }
}

}  // namespace stk
