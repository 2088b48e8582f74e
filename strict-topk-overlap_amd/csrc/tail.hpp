// Tail of the fused decode step: exact top-K of one query head's keys and
// the strict repair of its speculative attention, in one workgroup per head.
//
// Reference: strict_topk/gqa.py:145-161 (select_blocks), :164-193
// (repair_saved / repair_union) and gqa_light.py:10-92; the arithmetic of
// the saved repair is that of stk_gqa_repair.
//
// The tail runs on 32-64 workgroups, so its time is a chain of latencies;
// it is laid out around two dependent memory round trips:
//   1. the head's keys, its predicted row, its query row and every predicted
//      state (m, l, u) are requested together at entry;
//   2. the missed blocks' K/V tiles, once the top-K is known.
// In between: top-K by value bins (topk_bins.hpp), membership through an
// LDS map over block IDs (max predicted slot + 1, plus a selected flag), one
// packed scan that ranks the selected IDs and lists the misses (wave w
// takes misses w, w + 8, ...; their tile loads go out at once), and the
// hits' LSE partial sums from registers, per wave, with no further barrier
// before the merge.
//
// Cost model: a wave64 VALU instruction occupies a SIMD for 4 cycles and the
// 8 waves share 4 SIMDs, so every instruction on the path costs about 8
// cycles; the phases are kept short in instructions, LDS reads are issued
// together from clamped indices rather than under branches.
#pragma once

#include "topk_bins.hpp"
#include "tile2.hpp"

namespace stk {

constexpr int kTailThreads = 512;
constexpr int kTailWaves = kTailThreads / STK_WAVE;
constexpr int kTailMapN = 8192;      // block IDs covered by the LDS map
constexpr int kTailMaxK = 256;       // selected / predicted IDs per row
constexpr int kSelFlag = 1 << 30;    // map bit: block is selected

struct TailArgs {
  KV kv;                                  // q, k, v, hq, hkv, n, b, d
  const uint64_t* keys;                   // [hq, n]
  int k;                                  // selected per head
  int32_t* ids;                           // [hq, k] out, ascending
  const int32_t* p; int sp;               // predicted [hq, sp]
  const float* pm; const float* pl; const float* pu;   // predicted states
  int uni;                                // repair_union instead of saved
  float* out;                             // [hq, d]
  Paging pg;                              // PG: paged, batched KV
};

// KPT keys per thread (n <= 512 * KPT); RPT predicted-state rows per thread,
// four columns each (sp <= RPT * 2048 / D); ONE: a block is one token chunk.
// PG: paged, batched KV.  a.kv.n is then the key rows' and block table's
// width; the head's request has n <= a.kv.n blocks, of which min(k, n) are
// selected (the rest of the ID row is -1).  The pages of the row's blocks are
// loaded with the keys, so a selected block's page is known the moment the
// top-K names it, with no extra round trip before its tile.
template <typename T, int NCH, int UP, bool ONE, int KPT, int RPT, bool PG = false>
__device__ __forceinline__ void tail_head(const TailArgs& a) {
  using TT = TokTile<T, NCH, UP>;
  constexpr int D = TT::D;
  constexpr int TPR = D / 4;              // threads per state row (16-byte loads)
  constexpr int RG = kTailThreads / TPR;  // rows per pass of the state prefetch
  __shared__ int map[kTailMapN];
  __shared__ int sel[kTailMaxK], miss[kTailMaxK], pids[kTailMaxK];
  __shared__ float s_pm[kTailMaxK], s_pl[kTailMaxK];
  __shared__ TopkBinsLds tb;
  __shared__ int s_scan[kTailWaves];
  // the hits' partial sums, one row per wave (relative to the wave's max)
  __shared__ float s_hmax[kTailWaves], s_hl[kTailWaves];
  __shared__ __align__(16) float s_hu[kTailWaves][D];
  __shared__ float s_wm[kTailWaves], s_wl[kTailWaves], s_wu[kTailWaves][D];
  __shared__ int mtk[PG ? kTailMaxK : 1];   // PG: tokens of each listed miss
  const int h = xcd_remap(blockIdx.x, gridDim.x);   // a KV group's heads on one XCD
  const int nrow = a.kv.n, sp = a.sp;
  const int tid = threadIdx.x, w = wave_id();
  const int G = a.kv.hq / a.kv.hkv;
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
  // predicted (m, l) once per slot (to LDS below); u rows as 16-byte loads,
  // thread (rg, c4) holding columns 4*c4 .. 4*c4+3 of rows rg + RG*j
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
  // a predicted slot counts only with a state: a slot whose state is empty
  // (its block had no resident page when the front ran, as with a host-backed
  // cache) is recomputed like a miss when its block is selected
  auto fill_map = [&] {
    if (tid < sp && pid >= 0 && pid < n && pmv != -INFINITY) atomicMax(&map[pid], tid + 1);
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
  int pos = pre & 0xffff, mpos = pre >> 16;
  const int nm = total >> 16;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int idx = tid * KPT + i;
    if ((flags >> i) & 1u) {
      sel[pos++] = idx;
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
  // ---- round trip 2: wave w streams misses w, w + 8, ...; the first
  // tile's loads are issued before the hits' arithmetic
  const int kvh = PG ? kvp : h / G;
  const float scale = 1.0f / sqrtf((float)D);
  const T* K = reinterpret_cast<const T*>(a.kv.k);
  const T* V = reinterpret_cast<const T*>(a.kv.v);
  auto tile = [&](int x) {
    const size_t page = PG ? (size_t)miss[x] : (size_t)kvh * n + miss[x];
    return (page * a.kv.b) * D;
  };
  uint32_t kw[UP][TT::QW], vw[TT::CH][TT::VW];
  // the entry loads (u rows, query) returned during the top-K
  vm_drain();
  if (ONE && w < nm) t.load(K + tile(w), V + tile(w), 0, kw, vw);
  // the selected IDs go out behind the tile loads (stores count in the same
  // vector memory counter, so stores issued before the drain would hold it)
  for (int i = tid; i < a.k; i += kTailThreads)
    a.ids[(size_t)h * a.k + i] = (!PG || i < kk) ? sel[i] : -1;
  // ---- the hits' (or, for union, every predicted row's) partial LSE sums:
  // saved mode takes slot p when P[p] is selected and p is the highest slot
  // holding that block; union mode takes every slot.  Each wave sums its
  // rows relative to its own maximum (no barrier); the merge rescales.
  // (every LDS read is issued unconditionally, from clamped indices, so the
  // rows' reads go out together instead of one dependent round trip each)
  bool used[RPT];
  float um[RPT], ul[RPT];
  int pv[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int r = rg + RG * j;   // < 16 * RG <= 512
    const int rr = r < kTailMaxK ? r : 0;
    pv[j] = pids[rr];
    um[j] = s_pm[rr];
    ul[j] = s_pl[rr];
  }
  float hm = -INFINITY;
  const int nlast = n > 0 ? n - 1 : 0;
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int r = rg + RG * j;
    const bool inr = (pv[j] >= 0) & (pv[j] < n);
    const int mv = map[pv[j] < 0 ? 0 : (pv[j] > nlast ? nlast : pv[j])];
    const bool hit = ((mv & kSelFlag) != 0) & ((mv & ~kSelFlag) == r + 1);
    used[j] = (r < sp) & inr & ((a.uni != 0) | hit);
    hm = used[j] ? fmaxf(hm, um[j]) : hm;
  }
  hm = wave_max_u(hm);
  float hl = 0.f;
  float4 hu = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int r = rg + RG * j;
    const float wt = used[j] ? wexp(um[j], hm) : 0.f;
    // rows past sp were loaded from row 0 (or a stand-in buffer): zero them
    const float4 ur = r < sp ? uu[j] : make_float4(0.f, 0.f, 0.f, 0.f);
    hl += wt * ul[j];
    hu.x += wt * ur.x; hu.y += wt * ur.y; hu.z += wt * ur.z; hu.w += wt * ur.w;
  }
  // fold the row groups of this wave (lanes with the same columns)
  static_assert(TPR <= STK_WAVE, "state rows wider than a wave");
#pragma unroll
  for (int off = TPR; off < STK_WAVE; off <<= 1) {
    hl += __shfl_xor(hl, off);
    hu.x += __shfl_xor(hu.x, off); hu.y += __shfl_xor(hu.y, off);
    hu.z += __shfl_xor(hu.z, off); hu.w += __shfl_xor(hu.w, off);
  }
  if (lane_id() < TPR) *reinterpret_cast<float4*>(&s_hu[w][4 * c4]) = hu;
  if (lane_id() == 0) {
    s_hl[w] = hl;
    s_hmax[w] = hm;
  }
  // ---- the misses' states with the online softmax
  float m = -INFINITY, l = 0.f, acc[TT::DPL];
#pragma unroll
  for (int e = 0; e < TT::DPL; ++e) acc[e] = 0.f;
  for (int x = w; x < nm; x += kTailWaves) {
    // PG: a partly filled block weights only its first mtk[x] tokens
    const int lim = PG ? mtk[x] : a.kv.b;
    if constexpr (ONE) {
      if (x != w) t.load(K + tile(x), V + tile(x), 0, kw, vw);
      if (PG && lim < a.kv.b) t.update_part(qw, kw, vw, 0, lim, scale, m, l, acc);
      else t.template update<false, false>(qw, kw, vw, 0, a.kv.b, scale, m, l, acc);
    } else {
      for (int t0 = 0; t0 < lim; t0 += TT::CH) {
        t.load(K + tile(x), V + tile(x), t0, kw, vw);
        if (PG && t0 + TT::CH > lim) t.update_part(qw, kw, vw, t0, lim, scale, m, l, acc);
        else t.template update<false, false>(qw, kw, vw, t0, a.kv.b, scale, m, l, acc);
      }
    }
  }
  if (lane_id() == 0) {
    s_wm[w] = m;
    s_wl[w] = l;
  }
  t.store(s_wu[w], acc);
  __syncthreads();
  // ---- one LSE merge of the hits' partials and the waves' miss states
  if (tid < D) {
    float M = -INFINITY;
#pragma unroll
    for (int x = 0; x < kTailWaves; ++x) M = fmaxf(M, fmaxf(s_hmax[x], s_wm[x]));
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int x = 0; x < kTailWaves; ++x) {
      const float fh = wexp(s_hmax[x], M), f = wexp(s_wm[x], M);
      num += fh * s_hu[x][tid] + f * s_wu[x][tid];
      den += fh * s_hl[x] + f * s_wl[x];
    }
    a.out[(size_t)h * D + tid] = num / den;
  }
}

}  // namespace stk
