// Saved / union repair of one query head in one workgroup, laid out like the
// fused step's tail (tail.hpp) with the selected row given instead of
// computed: the drop-in repairs gqa.repair_saved / repair_union
// (strict_topk/gqa.py:164-193) and gqa_light.repair_saved_light
// (gqa_light.py:10-77) on the shapes the token tile covers.
//
// Two dependent memory round trips:
//   1. the selected and predicted rows, the query row and every predicted
//      state row (m, l and four columns of u per thread) are requested
//      together at entry;
//   2. the missed blocks' K/V tiles, once the membership map names them.
// In between: the LDS map (max predicted slot + 1 per block ID), one packed
// scan that lists the misses in selected-position order (wave w takes misses
// w, w + 8, ...), and the hits' LSE partial sums from registers while the
// tiles travel; then one merge.  Membership is the reference's: a selected
// block is a hit when some predicted slot holds it, and the hit takes the
// highest such slot's state (slot = max{j : P[j] == A[s]}, gqa.py:42);
// union mode merges every valid predicted slot and the misses.
#pragma once

#include "gqa_repair.hpp"
#include "tail.hpp"

namespace stk {

// Rows of predicted states per thread: four columns of a row per thread,
// 2048 / D rows per pass of the 512 threads.
inline int repair_fast_rpt(int sp, int d) {
  const int per_pass = kTailThreads * 4 / d;
  const int rows = (sp + per_pass - 1) / per_pass;
  return rows <= 4 ? 4 : (rows <= 16 ? 16 : 0);
}

template <typename T, int NCH, int UP, int RPT>
__device__ __forceinline__ void repair_fast_head(const GqaRepairArgs& a, int h) {
  using TT = TokTile<T, NCH, UP>;
  constexpr int D = TT::D;
  constexpr int TPR = D / 4;              // threads per state row (16-byte columns)
  constexpr int RG = kTailThreads / TPR;  // rows per pass of the state loads
  __shared__ int map[kTailMapN];
  __shared__ int miss[kTailMaxK], pids[kTailMaxK];
  __shared__ int s_scan[kTailWaves];
  __shared__ float s_hmax[kTailWaves], s_hl[kTailWaves];
  __shared__ __align__(16) float s_hu[kTailWaves][D];
  __shared__ float s_wm[kTailWaves], s_wl[kTailWaves], s_wu[kTailWaves][D];
  const int n = a.kv.n, sp = a.sp, sa = a.sa;
  const int tid = threadIdx.x, w = wave_id();
  const int G = a.kv.hq / a.kv.hkv;
  // ---- round trip 1: every load that does not depend on the membership
  // (64-bit IDs are range-checked before they are narrowed)
  const int64_t aid = load_id(a.a, a.atype, (int64_t)h * sa + (tid < sa ? tid : 0));
  const int64_t pid = load_id(a.p, a.ptype, (int64_t)h * sp + (tid < sp ? tid : 0));
  TT t;
  t.init();
  uint32_t qw[TT::QW];
  t.load_q(reinterpret_cast<const T*>(a.kv.q) + (size_t)h * D, qw);
  const int c4 = tid % TPR, rg = tid / TPR;
  float um[RPT], ul[RPT];
  float4 uu[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int r = rg + RG * j;
    const int64_t row = (int64_t)h * sp + (r < sp ? r : 0);
    um[j] = a.pm[row];
    ul[j] = a.pl[row];
    uu[j] = *reinterpret_cast<const float4*>(a.pu + row * D + 4 * c4);
  }
  for (int i = tid; i < n; i += kTailThreads) map[i] = 0;
  // every slot entry is written (-1 past sp): the sums below read entries
  // past sp, and LDS holds whatever an earlier workgroup left there
  const int myp = tid < sp && pid >= 0 && pid < n ? (int)pid : -1;
  if (tid < kTailMaxK) pids[tid] = myp;
  __syncthreads();
  if (myp >= 0 && myp < n) atomicMax(&map[myp], tid + 1);
  __syncthreads();
  // ---- the misses (valid selected IDs no predicted slot holds), listed in
  // selected-position order by one scan; the hits flagged in the map
  const int mya = tid < sa && aid >= 0 && aid < n ? (int)aid : -1;
  const bool av = mya >= 0 && mya < n;
  const int mv = map[av ? mya : 0];
  const bool ms = av && mv == 0;
  int nm;
  const int pos = block_excl_scan1(ms ? 1 : 0, s_scan, &nm);
  if (ms) miss[pos] = mya;
  if (av && mv != 0) atomicOr(&map[mya], kSelFlag);
  __syncthreads();
  // ---- round trip 2: wave w streams misses w, w + 8, ...
  const int kvh = h / G;
  const float scale = 1.0f / sqrtf((float)D);
  const T* K = reinterpret_cast<const T*>(a.kv.k);
  const T* V = reinterpret_cast<const T*>(a.kv.v);
  auto tile = [&](int x) { return (((size_t)kvh * n + miss[x]) * a.kv.b) * D; };
  uint32_t kw[UP][TT::QW], vw[TT::CH][TT::VW];
  vm_drain();   // the entry loads returned during the membership
  if (w < nm) t.load(K + tile(w), V + tile(w), 0, kw, vw);
  // ---- the hits' (union: every valid predicted row's) partial LSE sums,
  // each wave relative to its own maximum (the merge rescales)
  bool used[RPT];
  int pv[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int r = rg + RG * j;
    pv[j] = pids[r < kTailMaxK ? r : 0];
  }
  float hm = -INFINITY;
  const int nlast = n > 0 ? n - 1 : 0;
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int r = rg + RG * j;
    const bool inr = (pv[j] >= 0) & (pv[j] < n);
    const int mvv = map[pv[j] < 0 ? 0 : (pv[j] > nlast ? nlast : pv[j])];
    const bool hit = ((mvv & kSelFlag) != 0) & ((mvv & ~kSelFlag) == r + 1);
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
    // rows past sp were loaded from row 0: zero them
    const float4 ur = r < sp ? uu[j] : make_float4(0.f, 0.f, 0.f, 0.f);
    hl += wt * ul[j];
    hu.x += wt * ur.x; hu.y += wt * ur.y; hu.z += wt * ur.z; hu.w += wt * ur.w;
  }
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
    if (x != w) t.load(K + tile(x), V + tile(x), 0, kw, vw);
    t.template update<false, false>(qw, kw, vw, 0, a.kv.b, scale, m, l, acc);
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

// Launch the one-workgroup repair when it covers the shape (bf16 / fp16 Q/K/V
// 16-byte aligned, D in {64, 128, 256}, B of 16 or 32 tokens, N <= 8192, SA
// and SP <= 256, SP * D <= 32768 (16384 for D = 256 with B = 32), u 16-byte
// aligned); returns 1 (nothing launched) otherwise.
int launch_repair_fast(const GqaRepairArgs& g, int dtype, hipStream_t st);

}  // namespace stk
