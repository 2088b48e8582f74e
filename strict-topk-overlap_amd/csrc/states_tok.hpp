// Per-block softmax states on the token tile: the body of one workgroup of
// the states kernel (one wave per (query head, slot)).
//
// Reference: strict_topk/kernels.py:42-71 (_partial) and strict_topk/gqa.py:29-59
// (_partial): m = max logit, l = sum exp(logit - m), u = sum exp(logit - m) V
// with logits q.k / sqrt(D), query head h reading KV head h / G.
#pragma once

#include "tile2.hpp"

#ifndef STK_TOK_HT
#define STK_TOK_HT 1
#endif

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
constexpr int kTokHT = STK_TOK_HT;   // heads per pass over a resident token tile

// Token-tile states (shapes the token tile supports): one wave per
// (query head, slot).  GROUP: the wave owning block b (no lower head of its
// KV group lists b) computes the state of every head of the group whose row
// holds b, reading the K/V tile once; non-owners return.  Otherwise each wave
// computes its own slot, honouring the optional active mask (inactive slots
// get (-inf, 0, 0), kernels.py:42-71).
//
// ONE (B == CH): the block is loaded once and stays in registers while the
// heads are processed HT at a time; otherwise the block is streamed chunk by
// chunk for each batch of HT heads.  HT trades registers
// for passes: with HT = 1 the wave stays within 128 VGPRs, so four waves
// share a SIMD.
template <typename T, int NCH, int UP, typename I, bool GROUP, bool ONE,
          int HT = (GROUP ? kTokHT : 1)>
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
  int64_t bid;
  uint64_t found = 1ull << hl;
  if constexpr (GROUP) {
    // rows of the group that list b; G*S <= 256 IDs, 4 per lane, one pass
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
    found = 0ull;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int x = i * STK_WAVE + lane_id();
      if (x < total && v[i] == bid) found |= 1ull << (x / a.s);
    }
    for (int off = 1; off < STK_WAVE; off <<= 1) found |= __shfl_xor(found, off);
    if (found & ((1ull << hl) - 1ull)) return;   // a lower head owns this block
    found &= ~((1ull << hl) - 1ull);
  } else {
    bid = ids[item];
  }
  bool enabled = bid >= 0 && bid < a.n;
  if (!GROUP) {
    if (a.active_kind == 1) enabled = enabled && a.active[h] != 0;
    else if (a.active_kind == 2) enabled = enabled && a.active[item] != 0;
  }
  const int kv = h / G;
  TT t;
  t.init();
  const float scale = 1.0f / sqrtf((float)a.d);
  const size_t off = (((size_t)kv * a.n + (enabled ? (size_t)bid : 0)) * a.b) * a.d;
  const T* kb = reinterpret_cast<const T*>(a.k) + off;
  const T* vb = reinterpret_cast<const T*>(a.v) + off;
  uint32_t kw[UP][TT::QW], vw[TT::CH][TT::VW];
  if constexpr (ONE) t.load(kb, vb, 0, kw, vw);   // the whole block, once
  while (found) {
    int heads[HT];
    int nh = 0;
#pragma unroll
    for (int i = 0; i < HT; ++i) {
      heads[i] = hl;
      if (found) {
        int gg = __ffsll((long long)found) - 1;
        found &= found - 1;
        heads[i] = gg;
        nh = i + 1;
      }
    }
    uint32_t qw[HT][TT::QW];
    uint64_t pmask[HT];
    float m[HT], l[HT], acc[HT][TT::DPL];
#pragma unroll
    for (int i = 0; i < HT; ++i) {
      m[i] = -INFINITY;
      l[i] = 0.f;
#pragma unroll
      for (int e = 0; e < TT::DPL; ++e) acc[i][e] = 0.f;
      t.load_q(reinterpret_cast<const T*>(a.q) + (size_t)(g0 + heads[i]) * a.d, qw[i]);
      pmask[i] = 0ull;
      if constexpr (GROUP) {
        // rows of at most 64 IDs: positions of b, read with the query
        bool in = lane_id() < a.s;
        int64_t x = ld_or(ids, (int64_t)(g0 + heads[i]) * a.s + lane_id(), in, (I)-1);
        pmask[i] = __ballot(in && x == bid);
      }
    }
    if (enabled) {
      if constexpr (ONE) {
#pragma unroll
        for (int i = 0; i < HT; ++i)
          if (i < nh)
            t.template update<false, false>(qw[i], kw, vw, 0, a.b, scale, m[i], l[i], acc[i]);
      } else {
        for (int t0 = 0; t0 < a.b; t0 += TT::CH) {
          t.load(kb, vb, t0, kw, vw);
#pragma unroll
          for (int i = 0; i < HT; ++i)
            if (i < nh)
              t.template update<false, false>(qw[i], kw, vw, t0, a.b, scale, m[i], l[i], acc[i]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < HT; ++i) {
      if (i >= nh) continue;
      const int gg = heads[i];
      if (gg == hl) {
        if (lane_id() == 0) {
          a.m[item] = m[i];
          a.l[item] = l[i];
        }
        t.store(a.u + item * a.d, acc[i]);
        continue;
      }
      const int64_t rbase = (int64_t)(g0 + gg) * a.s;
      for (int p0 = 0; p0 < a.s; p0 += STK_WAVE) {
        int p = p0 + lane_id();
        uint64_t hits = pmask[i];
        if (p0 > 0) {
          int64_t x = ld_or(ids, rbase + p, p < a.s, (I)-1);
          hits = __ballot(p < a.s && x == bid);
        }
        while (hits) {
          int bit = __ffsll((long long)hits) - 1;
          hits &= hits - 1;
          int64_t row = rbase + p0 + bit;
          if (lane_id() == 0) {
            a.m[row] = m[i];
            a.l[row] = l[i];
          }
          t.store(a.u + row * a.d, acc[i]);
        }
      }
    }
  }
}

}  // namespace stk
