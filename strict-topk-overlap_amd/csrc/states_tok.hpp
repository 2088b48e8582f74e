// Per-block softmax states on the token tile: the body of one workgroup of
// the states kernel (one wave per (query head, slot)).
//
// Reference: strict_topk/kernels.py:42-71 (_partial) and strict_topk/gqa.py:29-59
// (_partial): m = max logit, l = sum exp(logit - m), u = sum exp(logit - m) V
// with logits q.k / sqrt(D), query head h reading KV head h / G.
#pragma once

#include "tile2.hpp"


namespace stk {

// Map a launch-order workgroup index to a logical index so that every XCD
// (workgroups are dealt round-robin over 8 XCDs) receives one contiguous
// range of logical workgroups.  Consecutive logical items share KV heads, so
// their tiles meet in the same XCD-local L2.
__device__ __forceinline__ int xcd_remap(int w, int total) {
  constexpr int X = 8;
  int xcd = w % X, r = w / X;
  int base = total / X, extra = total % X;
  int start = xcd * base + (xcd < extra ? xcd : extra);
  return start + r;
}

struct StatesArgs {
  const void* q; const void* k; const void* v;
  const void* ids; int itype;
  int hq, hkv, n, b, d, s;
  const uint8_t* active; int active_kind;     // 0 none, 1 per head, 2 per slot
  const void* pred; int ptype; int sp;        // slot mode: predicted rows
  int32_t* slot;                              // slot mode output [hq, s]
  float* m; float* l; float* u;               // [hq, s], [hq, s, d]
  const int32_t* slot_in; int slot_shared;    // hierarchical repair: skip hits
  int remap;
};

constexpr int kGrpHT = 4;   // heads sharing one loaded tile (generic-tile kernels)

// Up to 64 bits [o, o + len) of a 256-bit mask held as four wave-uniform words.
__device__ __forceinline__ uint64_t mask_bits(const uint64_t (&m)[4], int o, int len) {
  const int w = o >> 6, sh = o & 63;
  const uint64_t a = w == 0 ? m[0] : (w == 1 ? m[1] : (w == 2 ? m[2] : m[3]));
  const uint64_t b = w == 0 ? m[1] : (w == 1 ? m[2] : (w == 2 ? m[3] : 0ull));
  const uint64_t r = sh ? (a >> sh) | (b << (64 - sh)) : a;
  return len >= 64 ? r : (r & ((1ull << len) - 1ull));
}

// Token-tile states (shapes the token tile supports): one wave per
// (query head, slot).  GROUP: the wave owning block b (no lower head of its
// KV group lists b) computes the state of every head of the group whose row
// holds b, reading the K/V tile once; non-owners return.  Otherwise each wave
// computes its own slot, honouring the optional active mask (inactive slots
// get (-inf, 0, 0), kernels.py:42-71).
//
// Dependent memory round trips are what a wave waits for when HBM queues
// are full, so there are two: (1) the group's IDs and the wave's own query
// row, (2) the K/V tile.  The rows that list b come from ballots over the
// IDs of round trip 1, so writing the states needs no further ID loads; a
// further head's query row is loaded while the previous head finishes.  ONE (B == CH): the block is loaded once
// and stays in registers while the heads are processed in turn (one head at
// a time keeps the wave within 128 VGPRs: four waves per SIMD); otherwise
// each head streams the block chunk by chunk.
template <typename T, int NCH, int UP, typename I, bool GROUP, bool ONE>
__device__ __forceinline__ void states_tok_wg(const StatesArgs& a, int wg) {
  using TT = TokTile<T, NCH, UP>;
  const int waves = blockDim.x / STK_WAVE;
  int64_t item = (int64_t)wg * waves + wave_id();
  if (item >= (int64_t)a.hq * a.s) return;
  const I* ids = reinterpret_cast<const I*>(a.ids);
  const int h = (int)(item / a.s);
  const int j = (int)(item - (int64_t)h * a.s);
  const int G = a.hq / a.hkv;
  const int hl = h % G;
  const int g0 = h - hl;
  TT t;
  t.init();
  const T* qg = reinterpret_cast<const T*>(a.q) + (size_t)g0 * a.d;
  uint32_t qw[TT::QW];
  t.load_q(qg + (size_t)hl * a.d, qw);   // own query row, with the IDs
  int64_t bid;
  uint64_t found = 1ull << hl;           // heads of the group listing b
  uint64_t rows[4] = {0ull, 0ull, 0ull, 0ull};   // ID == b over the group's G*S IDs
  if constexpr (GROUP) {
    // the group's G*S <= 256 IDs, 4 per lane, in one pass
    const int total = G * a.s;
    const I* grp = ids + (int64_t)g0 * a.s;
    int64_t v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int x = i * STK_WAVE + lane_id();
      v[i] = ld_or(grp, (int64_t)x, x < total, (I)-1);
    }
    const int xb = hl * a.s + j;
    const int ib = xb / STK_WAVE, lb = xb % STK_WAVE;
    int64_t pick = v[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) pick = ib == i ? v[i] : pick;
    bid = __shfl(pick, lb);
#pragma unroll
    for (int i = 0; i < 4; ++i) rows[i] = __ballot(i * STK_WAVE + lane_id() < total && v[i] == bid);
    found = 0ull;
    for (int r = 0; r < G; ++r)
      if (mask_bits(rows, r * a.s, a.s < 64 ? a.s : 64) != 0ull ||
          (a.s > 64 && mask_bits(rows, r * a.s + 64, a.s - 64) != 0ull))
        found |= 1ull << r;
    if (found & ((1ull << hl) - 1ull)) return;   // a lower head owns this block
  } else {
    bid = ids[item];
  }
  bool enabled = bid >= 0 && bid < a.n;
  if (!GROUP) {
    if (a.active_kind == 1) enabled = enabled && a.active[h] != 0;
    else if (a.active_kind == 2) enabled = enabled && a.active[item] != 0;
  }
  const int kv = h / G;
  const float scale = 1.0f / sqrtf((float)a.d);
  const size_t off = (((size_t)kv * a.n + (enabled ? (size_t)bid : 0)) * a.b) * a.d;
  const T* kb = reinterpret_cast<const T*>(a.k) + off;
  const T* vb = reinterpret_cast<const T*>(a.v) + off;
  uint32_t kw[UP][TT::QW], vw[TT::CH][TT::VW];
  if constexpr (ONE) {
    t.load(kb, vb, 0, kw, vw);   // the whole block, once
    // all of the tile's loads are issued before any arithmetic (the
    // scheduler would otherwise sink the V loads below the Q.K products)
    __builtin_amdgcn_sched_barrier(0);
  }
  // heads after the owner, lowest first
  uint64_t rest = found & ~(1ull << hl);
  int cur = hl;
  while (true) {
    float m = -INFINITY, l = 0.f, acc[TT::DPL];
#pragma unroll
    for (int e = 0; e < TT::DPL; ++e) acc[e] = 0.f;
    const int nxt = rest ? __ffsll((long long)rest) - 1 : cur;
    if constexpr (ONE) {
      // opaque tile words: the value conversions stay inside the head loop
      // (hoisted out of it they would hold every token's FP32 values)
#pragma unroll
      for (int i = 0; i < TT::CH; ++i)
#pragma unroll
        for (int w = 0; w < TT::VW; ++w) asm volatile("" : "+v"(vw[i][w]));
      float s[UP];
      t.scores(qw, kw, 0, a.b, scale, s);
      // the next head's query loads into the registers just freed, hidden
      // behind this head's softmax and P.V
      if (rest) t.load_q(qg + (size_t)nxt * a.d, qw);
      if (enabled) t.template accumulate<false, false>(s, vw, m, l, acc);
    } else {
      if (enabled) {
        for (int t0 = 0; t0 < a.b; t0 += TT::CH) {
          t.load(kb, vb, t0, kw, vw);
          t.template update<false, false>(qw, kw, vw, t0, a.b, scale, m, l, acc);
        }
      }
      if (rest) t.load_q(qg + (size_t)nxt * a.d, qw);
    }
    if (cur == hl) {
      if (lane_id() == 0) {
        a.m[item] = m;
        a.l[item] = l;
      }
      t.store(a.u + item * a.d, acc);
    } else {
      const int64_t rbase = (int64_t)(g0 + cur) * a.s;
      for (int p0 = 0; p0 < a.s; p0 += STK_WAVE) {
        const int len = a.s - p0 < 64 ? a.s - p0 : 64;
        uint64_t hits = mask_bits(rows, cur * a.s + p0, len);
        while (hits) {
          const int bit = __ffsll((long long)hits) - 1;
          hits &= hits - 1;
          const int64_t row = rbase + p0 + bit;
          if (lane_id() == 0) {
            a.m[row] = m;
            a.l[row] = l;
          }
          t.store(a.u + row * a.d, acc);
        }
      }
    }
    if (!rest) break;
    rest &= rest - 1;
    cur = nxt;
  }
}

}  // namespace stk
