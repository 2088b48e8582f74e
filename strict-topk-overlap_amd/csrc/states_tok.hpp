// Per-block softmax states on the token tile: the body of one workgroup of
// the states kernel (one wave per (query head, slot)).
//
// Reference: strict_topk/kernels.py:42-71 (_partial) and strict_topk/gqa.py:29-59
// (_partial): m = max logit, l = sum exp(logit - m), u = sum exp(logit - m) V
// with logits q.k / sqrt(D), query head h reading KV head h / G.
#pragma once

#include "tile2.hpp"


namespace stk {

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
  // hierarchical exact / repair (grouped pack kernel): one merged state per
  // pack of 32 / B positions into m, l, u [hq, packs]; with slot_in, a hit's
  // state is the prediction's (pm, pl, pu [hq, psp(, d)]) at its slot
  int combine;
  const float* pm; const float* pl; const float* pu; int psp;
  uint32_t* tflag;                            // SIG: [hq * s], set once an item's state is published
  int drop;                                   // SIG, tests only: publish no flag
};

constexpr int kGrpHT = 4;   // heads sharing one loaded tile (generic-tile kernels)

// Token-tile states (shapes the token tile supports): one wave per
// (query head, slot), honouring the optional active mask (inactive slots and
// invalid IDs get (-inf, 0, 0), kernels.py:42-71).
//
// The wave waits on two dependent memory round trips: (1) its block ID with
// its query row, (2) the K/V tile.  Query heads of one KV group that list
// the same block each read its tile; the items of a KV group are contiguous
// and land on one XCD (xcd_remap), so the repeated reads are served by that
// XCD's L2.  Measured on MI355X this beats computing a block once for all
// the heads that list it: every wave then carries exactly one head's work,
// and the first round trip is one ID instead of the group's rows.
//
// ONE (B == CH): the block is one token chunk, loaded once; otherwise the
// block is streamed chunk by chunk.  PG: paged, batched KV (a.n is the block
// table's row width; an ID at or past its request's block count, or on an
// invalid page, gets the empty state).
// SIG (the one-launch step): the state is stored agent-coherent and, once
// the wave's stores have completed, the item's flag is set.
template <typename T, int NCH, int UP, typename I, bool ONE, bool PG = false, bool SIG = false>
__device__ __forceinline__ void states_tok_wg(const StatesArgs& a, int wg,
                                              const Paging& pg = Paging{}) {
  using TT = TokTile<T, NCH, UP>;
  const int waves = blockDim.x / STK_WAVE;
  const int64_t item = (int64_t)wg * waves + wave_id();
  if (item >= (int64_t)a.hq * a.s) return;
  const int h = (int)(item / a.s);
  TT t;
  t.init();
  uint32_t qw[TT::QW];
  t.load_q(reinterpret_cast<const T*>(a.q) + (size_t)h * a.d, qw);
  const int64_t bid = reinterpret_cast<const I*>(a.ids)[item];
  const int kv = h / (a.hq / a.hkv);
  // PG: the row's block count comes with the ID; the table entry needs only
  // the ID (bounded by the table width), then the tile needs the page
  const int nv = PG ? pg_blocks(pg, kv, a.n) : a.n;
  const int rtok = PG ? pg_row_tokens(pg, kv) : 0;
  const bool inrow = bid >= 0 && bid < a.n;
  // PG: tokens of the block holding data (the request's last block may be
  // partly filled; a block with none has the empty state)
  const int bval = PG ? pg_block_tokens(rtok, bid, a.b) : a.b;
  bool enabled = inrow && bid < nv && (!PG || bval > 0);
  if (a.active_kind == 1) enabled = enabled && a.active[h] != 0;
  else if (a.active_kind == 2) enabled = enabled && a.active[item] != 0;
  const float scale = 1.0f / sqrtf((float)a.d);
  size_t page;
  if constexpr (PG) {
    const int pgi = pg_page(pg, kv, a.n, bid, inrow);
    enabled = enabled && pgi >= 0;
    page = enabled ? (size_t)pgi : 0;
  } else {
    page = (size_t)kv * a.n + (enabled ? (size_t)bid : 0);
  }
  const size_t off = (page * a.b) * a.d;
  const T* kb = reinterpret_cast<const T*>(a.k) + off;
  const T* vb = reinterpret_cast<const T*>(a.v) + off;
  float m = -INFINITY, l = 0.f, acc[TT::DPL];
#pragma unroll
  for (int e = 0; e < TT::DPL; ++e) acc[e] = 0.f;
  uint32_t kw[UP][TT::QW], vw[TT::CH][TT::VW];
  if constexpr (ONE) {
    t.load(kb, vb, 0, kw, vw);   // the whole block
    // all of the tile's loads are issued before any arithmetic (the
    // scheduler would otherwise sink the V loads below the Q.K products)
    __builtin_amdgcn_sched_barrier(0);
    if (enabled) {
      if (PG && bval < a.b) t.update_part(qw, kw, vw, 0, bval, scale, m, l, acc);
      else t.template update<false, false>(qw, kw, vw, 0, a.b, scale, m, l, acc);
    }
  } else if (enabled) {
    for (int t0 = 0; t0 < bval; t0 += TT::CH) {
      t.load(kb, vb, t0, kw, vw);
      if (PG && t0 + TT::CH > bval) t.update_part(qw, kw, vw, t0, bval, scale, m, l, acc);
      else t.template update<false, false>(qw, kw, vw, t0, a.b, scale, m, l, acc);
    }
  }
  if constexpr (SIG) {
    if (lane_id() == 0) {
      st_agent(a.m + item, m);
      st_agent(a.l + item, l);
    }
    t.store_agent(a.u + item * a.d, acc);
    wait_stores();
    if (!a.drop && lane_id() == 0) st_agent(a.tflag + item, 1u);
  } else {
    if (lane_id() == 0) {
      a.m[item] = m;
      a.l[item] = l;
    }
    t.store(a.u + item * a.d, acc);
  }
}

}  // namespace stk
