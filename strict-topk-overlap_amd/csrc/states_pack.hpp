// Per-block softmax states for small blocks (B = 4 or 8 tokens): one wave per
// (query head, pack of 32 / B consecutive positions of its ID row).
//
// Reference: strict_topk/gqa_hierarchical.py:22-61 (_packed_partials, PACK = 8
// blocks per program when B <= 8) and strict_topk/kernels.py:42-71 /
// gqa.py:29-59 (_partial): m = max logit, l = sum exp(logit - m),
// u = sum exp(logit - m) V per block, logits q.k / sqrt(D).
//
// The 32 tokens of a pack form one token-tile chunk (TokTile<T, NCH, 2>):
// four lanes per token row for Q.K, token slots 0..15 in two passes.  A
// B = 4 block is then one 16-lane DPP row of one pass, a B = 8 block two
// rows, so the per-block max and sum are row reductions (plus one exchange
// between the two rows for B = 8).  P.V keeps one accumulator per block;
// each token's weight is broadcast by readlane.  Memory round trips: (1) the
// pack's block IDs (each lane loads the IDs its own K rows need) with the
// query row, (2) the 32 K rows and 32 V rows.  Positions past the row end,
// skipped hits (slot_in >= 0) and inactive slots are handled as in the
// generic kernel; invalid IDs give (-inf, 0, 0) and read block 0's memory.
#pragma once

#include "states_tok.hpp"

namespace stk {

template <typename T, int NCH, int BB, typename I>
__device__ __forceinline__ void states_pack_wg(const StatesArgs& a, int wg) {
  using TT = TokTile<T, NCH, 2>;
  static_assert(BB == 4 || BB == 8, "packed blocks hold 4 or 8 tokens");
  constexpr int PB = TT::CH / BB;        // blocks per pack
  constexpr int D = TT::D;
  const int waves = blockDim.x / STK_WAVE;
  const int packs = (a.s + PB - 1) / PB;
  const int64_t item = (int64_t)wg * waves + wave_id();
  if (item >= (int64_t)a.hq * packs) return;
  const int h = (int)(item / packs);
  const int p0 = (int)(item - (int64_t)h * packs) * PB;
  const int G = a.hq / a.hkv;
  const int kv = h / G;
  const I* ids = reinterpret_cast<const I*>(a.ids) + (int64_t)h * a.s;
  TT t;
  t.init();
  // ---- round trip 1: block IDs (per lane, those of its own K rows, and
  // lane j < PB holding position p0 + j) and the query row
  int64_t kid[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int pos = p0 + (t.slot + 16 * u) / BB;
    kid[u] = ld_or(ids, (int64_t)pos, pos < a.s, (I)-1);
  }
  const int jl = lane_id() < PB ? lane_id() : 0;
  const int64_t lid = ld_or(ids, (int64_t)(p0 + jl), lane_id() < PB && p0 + jl < a.s, (I)-1);
  uint32_t qw[TT::QW];
  t.load_q(reinterpret_cast<const T*>(a.q) + (size_t)h * D, qw);
  // per-position flags (lane j < PB): write the state, and compute it
  bool write = lane_id() < PB && p0 + jl < a.s;
  if (write && a.slot_in)
    write = a.slot_in[(int64_t)(a.slot_shared ? 0 : h) * a.s + p0 + jl] < 0;
  bool live = write && lid >= 0 && lid < a.n;
  if (a.active_kind == 1) live = live && a.active[h] != 0;
  else if (a.active_kind == 2) live = live && write && a.active[(int64_t)h * a.s + p0 + jl] != 0;
  const uint64_t wmask = __ballot(write);
  if (wmask == 0ull) return;   // every position of the pack is a skipped hit or past the end
  const uint64_t lmask = __ballot(live);
  // ---- round trip 2: the pack's K rows (this lane's tokens) and V rows
  const T* K = reinterpret_cast<const T*>(a.k);
  const T* V = reinterpret_cast<const T*>(a.v);
  uint32_t kw[2][TT::QW], vw[TT::CH][TT::VW];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int tok = t.slot + 16 * u;
    const bool ok = kid[u] >= 0 && kid[u] < a.n;
    const T* row = K + ((((size_t)kv * a.n + (ok ? (size_t)kid[u] : 0)) * BB + tok % BB) * D);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const uint4 x = *reinterpret_cast<const uint4*>(row + t.kdim(c));
      kw[u][4 * c + 0] = x.x; kw[u][4 * c + 1] = x.y; kw[u][4 * c + 2] = x.z;
      kw[u][4 * c + 3] = x.w;
    }
  }
#pragma unroll
  for (int j = 0; j < PB; ++j) {
    const int64_t bj = __builtin_amdgcn_readlane((int)lid, j);   // IDs fit in 32 bits here
    const bool ok = (lmask >> j) & 1ull;
    const T* vb = V + (((size_t)kv * a.n + (ok ? (size_t)bj : 0)) * BB) * D + lane_id() * TT::DPL;
#pragma unroll
    for (int r = 0; r < BB; ++r) {
      const T* row = vb + (size_t)r * D;
      const int i = j * BB + r;
      if constexpr (TT::DPL * sizeof(T) == 2) {
        vw[i][0] = *reinterpret_cast<const uint16_t*>(row);
      } else if constexpr (TT::DPL * sizeof(T) == 4) {
        vw[i][0] = *reinterpret_cast<const uint32_t*>(row);
      } else if constexpr (TT::DPL * sizeof(T) == 8) {
        const uint2 x = *reinterpret_cast<const uint2*>(row);
        vw[i][0] = x.x; vw[i][1] = x.y;
      } else {
        const uint4 x = *reinterpret_cast<const uint4*>(row);
        vw[i][0] = x.x; vw[i][1] = x.y; vw[i][2] = x.z; vw[i][3] = x.w;
      }
    }
  }
  // every K and V load is in flight before the first arithmetic (the
  // scheduler would otherwise sink the V loads below the Q.K products and
  // pay a second memory round trip)
  __builtin_amdgcn_sched_barrier(0);
  // ---- logits of this lane's two tokens (-inf for blocks not computed)
  const float scale = 1.0f / sqrtf((float)D);
  float s[2];
  t.scores(qw, kw, 0, TT::CH, scale, s);
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int j = (t.slot + 16 * u) / BB;
    if (!((lmask >> j) & 1ull)) s[u] = -INFINITY;
  }
  // ---- per-block max and sum: a 16-lane row per 4 tokens (quads hold one
  // token), two rows per 8 tokens
  float mb[2], w[2], lb[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    float x = s[u];
    x = fmaxf(x, dpp<0x141>(x, x));
    x = fmaxf(x, dpp<0x140>(x, x));
    if constexpr (BB == 8) x = fmaxf(x, __shfl_xor(x, 16));
    mb[u] = x;
    w[u] = wexp(s[u], x);
    float y = t.part == 0 ? w[u] : 0.f;
    y += dpp<0xB1>(0.f, y);
    y += dpp<0x4E>(0.f, y);
    y += dpp<0x141>(0.f, y);
    y += dpp<0x140>(0.f, y);
    if constexpr (BB == 8) y += __shfl_xor(y, 16);
    lb[u] = y;
  }
  // ---- P.V, one accumulator per block
  float acc[PB][TT::DPL];
#pragma unroll
  for (int j = 0; j < PB; ++j)
#pragma unroll
    for (int e = 0; e < TT::DPL; ++e) acc[j][e] = 0.f;
#pragma unroll
  for (int i = 0; i < TT::CH; ++i) {
    const int u = i / 16, src = (i % 16) * 4;
    const float wt = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w[u]), src));
    float v[TT::DPL];
    t.vals(vw, i, v);
#pragma unroll
    for (int e = 0; e < TT::DPL; ++e) acc[i / BB][e] += wt * v[e];
  }
  // ---- states of the pack's positions
#pragma unroll
  for (int j = 0; j < PB; ++j) {
    if (!((wmask >> j) & 1ull)) continue;
    const int u = (j * BB) / 16, src = ((j * BB) % 16) * 4;
    const int64_t row = (int64_t)h * a.s + p0 + j;
    if (lane_id() == 0) {
      a.m[row] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mb[u]), src));
      a.l[row] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lb[u]), src));
    }
    t.store(a.u + row * D, acc[j]);
  }
}

// The same packed states for HG query heads of one KV group per wave.  When
// the HG heads list the same IDs at the pack's positions (a selection shared
// by the group, as gqa_hierarchical.repair_saved_shared assumes, or any rows
// that happen to agree there), the pack's 32 K rows and 32 V rows are loaded
// once and the heads are computed in turn from registers; otherwise each head
// loads its own rows.  Items are ordered (KV head, pack, head group), so the
// waves sharing a pack are adjacent and land on one XCD.
template <typename T, int NCH, int BB, typename I, int HG, bool COMB = false>
__device__ __forceinline__ void states_pack_grp_wg(const StatesArgs& a, int wg) {
  using TT = TokTile<T, NCH, 2>;
  static_assert(BB == 4 || BB == 8, "packed blocks hold 4 or 8 tokens");
  constexpr int PB = TT::CH / BB;        // blocks per pack
  constexpr int D = TT::D;
  static_assert(HG * PB <= STK_WAVE, "one ID per lane for the group");
  const int waves = blockDim.x / STK_WAVE;
  const int packs = (a.s + PB - 1) / PB;
  const int G = a.hq / a.hkv;
  const int hgs = G / HG;
  // COMB: a workgroup takes four consecutive packs of one head group (a wave
  // past the last pack computes an empty state) and merges them in LDS;
  // workgroups are ordered (KV head, four packs, head group), so the head
  // groups of the same packs are adjacent and land on one XCD
  const int pgroups = (packs + 3) / 4;
  int hg, pack, kv;
  if constexpr (COMB) {
    hg = wg % hgs;
    const int rest = wg / hgs;
    pack = (rest % pgroups) * 4 + wave_id();
    kv = rest / pgroups;
  } else {
    const int64_t item = (int64_t)wg * waves + wave_id();
    if (item >= (int64_t)a.hkv * packs * hgs) return;
    hg = (int)(item % hgs);
    const int64_t rest = item / hgs;
    pack = (int)(rest % packs);
    kv = (int)(rest / packs);
  }
  const int h0 = kv * G + hg * HG;
  const int p0 = pack * PB;
  const I* ids = reinterpret_cast<const I*>(a.ids);
  // COMB: the four waves' pack states, merged after the head loop
  __shared__ float s_cu[COMB ? 4 : 1][COMB ? HG : 1][COMB ? D : 1];
  __shared__ float s_cm[COMB ? 4 : 1][COMB ? HG : 1], s_cl[COMB ? 4 : 1][COMB ? HG : 1];
  TT t;
  t.init();
  // ---- round trip 1: the group's IDs at the pack (lane i * PB + j holds
  // head h0 + i, position p0 + j), the first head's query row
  const int gi = lane_id() / PB, gj = lane_id() % PB;
  const bool gin = lane_id() < HG * PB && p0 + gj < a.s;
  const int64_t gid = ld_or(ids, (int64_t)(h0 + (gi < HG ? gi : 0)) * a.s + p0 + gj, gin, (I)-1);
  uint32_t qw[TT::QW];
  t.load_q(reinterpret_cast<const T*>(a.q) + (size_t)h0 * D, qw);
  // hierarchical repair: the slots of the same (head, position) pairs come
  // in the same round trip; a hit's tile is not needed, and its rows are
  // read from block 0 (one cached line) instead
  const int gsl = a.slot_in && gin
                      ? a.slot_in[(int64_t)(a.slot_shared ? 0 : h0 + (gi < HG ? gi : 0)) * a.s +
                                  p0 + gj]
                      : -1;
  const int64_t ref = __shfl(gid, gj);
  const int sref = __shfl(gsl, gj);
  // one tile load for the group when the heads agree on the IDs and on which
  // of them are hits
  const bool same = __ballot(lane_id() < HG * PB && (gid != ref || gsl != sref)) == 0ull;
  const T* K = reinterpret_cast<const T*>(a.k);
  const T* V = reinterpret_cast<const T*>(a.v);
  uint32_t kw[2][TT::QW], vw[TT::CH][TT::VW];
  const float scale = 1.0f / sqrtf((float)D);
  // K/V rows of the pack for head i's IDs (lanes hold the IDs of their rows)
  auto load_tile = [&](int i) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int tok = t.slot + 16 * u;
      // both shuffles run in every lane: a cross-lane read inside a
      // condition would see the lanes the condition turned off as zeros
      const int64_t bid = __shfl(gid, i * PB + tok / BB);
      const int bsl = __shfl(gsl, i * PB + tok / BB);
      const bool ok = bid >= 0 && bid < a.n && bsl < 0;
      const T* row = K + ((((size_t)kv * a.n + (ok ? (size_t)bid : 0)) * BB + tok % BB) * D);
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const uint4 x = *reinterpret_cast<const uint4*>(row + t.kdim(c));
        kw[u][4 * c + 0] = x.x; kw[u][4 * c + 1] = x.y; kw[u][4 * c + 2] = x.z;
        kw[u][4 * c + 3] = x.w;
      }
    }
#pragma unroll
    for (int j = 0; j < PB; ++j) {
      const int64_t bj = __builtin_amdgcn_readlane((int)gid, i * PB + j);   // IDs fit in 32 bits
      const bool ok = bj >= 0 && bj < a.n && __builtin_amdgcn_readlane(gsl, i * PB + j) < 0;
      const T* vb = V + (((size_t)kv * a.n + (ok ? (size_t)bj : 0)) * BB) * D + lane_id() * TT::DPL;
#pragma unroll
      for (int r = 0; r < BB; ++r) {
        const T* row = vb + (size_t)r * D;
        const int x = j * BB + r;
        if constexpr (TT::DPL * sizeof(T) == 2) {
          vw[x][0] = *reinterpret_cast<const uint16_t*>(row);
        } else if constexpr (TT::DPL * sizeof(T) == 4) {
          vw[x][0] = *reinterpret_cast<const uint32_t*>(row);
        } else if constexpr (TT::DPL * sizeof(T) == 8) {
          const uint2 y = *reinterpret_cast<const uint2*>(row);
          vw[x][0] = y.x; vw[x][1] = y.y;
        } else {
          const uint4 y = *reinterpret_cast<const uint4*>(row);
          vw[x][0] = y.x; vw[x][1] = y.y; vw[x][2] = y.z; vw[x][3] = y.w;
        }
      }
    }
  };
  if (same) load_tile(0);
  for (int i = 0; i < HG; ++i) {
    const int h = h0 + i;
    if (!same) load_tile(i);
    // all of this head's loads are in flight before its arithmetic
    __builtin_amdgcn_sched_barrier(0);
    // per-position flags (lane j < PB): write the state, and compute it
    const int jl = lane_id() < PB ? lane_id() : 0;
    const int64_t lid = __shfl(gid, i * PB + jl);
    const bool inr = lane_id() < PB && p0 + jl < a.s;
    const int slr = __shfl(gsl, i * PB + jl);   // in every lane (see load_tile)
    const int sl = inr ? slr : -1;
    const bool write = inr && sl < 0;
    bool live = write && lid >= 0 && lid < a.n;
    if (a.active_kind == 1) live = live && a.active[h] != 0;
    else if (a.active_kind == 2) live = live && a.active[(int64_t)h * a.s + p0 + jl] != 0;
    const uint64_t wmask = __ballot(write);
    const uint64_t lmask = __ballot(live);
    // combine mode: lane j < PB requests the m, l of position j's hit with
    // the tiles; the hits' u rows are read after the arithmetic (requesting
    // them here would keep 16 more registers live across it)
    // (a slot past the prediction's rows is no hit and reads nothing)
    const bool hit = COMB && a.pm != nullptr && inr && sl >= 0 && sl < a.psp;
    const uint64_t hmask = __ballot(hit);
    float hm = -INFINITY, hl = 0.f;
    if (hit) {
      const int64_t prow = (int64_t)h * a.psp + sl;
      hm = a.pm[prow];
      hl = a.pl[prow];
    }
    float s[2];
    t.scores(qw, kw, 0, TT::CH, scale, s);
    // the next head's query row, loaded while this head finishes
    if (i + 1 < HG) t.load_q(reinterpret_cast<const T*>(a.q) + (size_t)(h + 1) * D, qw);
    if (wmask == 0ull && !COMB) continue;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = (t.slot + 16 * u) / BB;
      if (!((lmask >> j) & 1ull)) s[u] = -INFINITY;
    }
    float mb[2], w[2], lb[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float x = s[u];
      x = fmaxf(x, dpp<0x141>(x, x));
      x = fmaxf(x, dpp<0x140>(x, x));
      if constexpr (BB == 8) x = fmaxf(x, __shfl_xor(x, 16));
      mb[u] = x;
      w[u] = wexp(s[u], x);
      float y = t.part == 0 ? w[u] : 0.f;
      y += dpp<0xB1>(0.f, y);
      y += dpp<0x4E>(0.f, y);
      y += dpp<0x141>(0.f, y);
      y += dpp<0x140>(0.f, y);
      if constexpr (BB == 8) y += __shfl_xor(y, 16);
      lb[u] = y;
    }
    float acc[PB][TT::DPL];
#pragma unroll
    for (int j = 0; j < PB; ++j)
#pragma unroll
      for (int e = 0; e < TT::DPL; ++e) acc[j][e] = 0.f;
#pragma unroll
    for (int x = 0; x < TT::CH; ++x) {
      const int u = x / 16, src = (x % 16) * 4;
      const float wt = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w[u]), src));
      float v[TT::DPL];
      t.vals(vw, x, v);
#pragma unroll
      for (int e = 0; e < TT::DPL; ++e) acc[x / BB][e] += wt * v[e];
    }
    if constexpr (COMB) {
      // a hit's u row replaces its (empty) computed accumulator
#pragma unroll
      for (int j = 0; j < PB; ++j) {
        if ((hmask >> j) & 1ull) {
          const int sj = __builtin_amdgcn_readlane(sl, j);
          const float* ur = a.pu + ((int64_t)h * a.psp + sj) * D + lane_id() * TT::DPL;
#pragma unroll
          for (int e = 0; e < TT::DPL; ++e) acc[j][e] = ur[e];
        }
      }
      // one merged state for the pack: computed blocks, hits from the
      // prediction, the rest empty
      float mj[PB], lj[PB];
      float M = -INFINITY;
#pragma unroll
      for (int j = 0; j < PB; ++j) {
        const int u = (j * BB) / 16, src = ((j * BB) % 16) * 4;
        const bool hj = (hmask >> j) & 1ull, comp = (lmask >> j) & 1ull;
        const float cm = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mb[u]), src));
        const float cl = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lb[u]), src));
        const float pmj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, hm), j));
        const float plj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, hl), j));
        mj[j] = hj ? pmj : (comp ? cm : -INFINITY);
        lj[j] = hj ? plj : (comp ? cl : 0.f);
        M = fmaxf(M, mj[j]);
      }
      float Z = 0.f, U[TT::DPL];
#pragma unroll
      for (int e = 0; e < TT::DPL; ++e) U[e] = 0.f;
#pragma unroll
      for (int j = 0; j < PB; ++j) {
        const float f = wexp(mj[j], M);   // 0 for an empty position
        Z += f * lj[j];
#pragma unroll
        for (int e = 0; e < TT::DPL; ++e) U[e] += f * acc[j][e];
      }
      if (lane_id() == 0) {
        s_cm[wave_id()][i] = M;
        s_cl[wave_id()][i] = Z;
      }
#pragma unroll
      for (int e = 0; e < TT::DPL; ++e) s_cu[wave_id()][i][lane_id() * TT::DPL + e] = U[e];
      continue;
    }
#pragma unroll
    for (int j = 0; j < PB; ++j) {
      if (!((wmask >> j) & 1ull)) continue;
      const int u = (j * BB) / 16, src = ((j * BB) % 16) * 4;
      const int64_t row = (int64_t)h * a.s + p0 + j;
      if (lane_id() == 0) {
        a.m[row] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mb[u]), src));
        a.l[row] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lb[u]), src));
      }
      t.store(a.u + row * D, acc[j]);
    }
  }
  if constexpr (COMB) {
    // one state per (head, four packs): wave x merges head x of the group
    __syncthreads();
    const int x = wave_id();
    if (x < HG) {
      float M = -INFINITY;
#pragma unroll
      for (int y = 0; y < 4; ++y) M = fmaxf(M, s_cm[y][x]);
      float L = 0.f, U[TT::DPL];
#pragma unroll
      for (int e = 0; e < TT::DPL; ++e) U[e] = 0.f;
#pragma unroll
      for (int y = 0; y < 4; ++y) {
        const float f = wexp(s_cm[y][x], M);   // 0 for an empty pack
        L += f * s_cl[y][x];
#pragma unroll
        for (int e = 0; e < TT::DPL; ++e) U[e] += f * s_cu[y][x][lane_id() * TT::DPL + e];
      }
      const int64_t row = (int64_t)(h0 + x) * pgroups + pack / 4;
      if (lane_id() == 0) {
        a.m[row] = M;
        a.l[row] = L;
      }
      t.store(a.u + row * D, U);
    }
  }
}

// Packed token tile shape for (dtype, D, B): NCH, or 0 when unsupported.
inline int pack_nch(int dtype, int d, int b, uintptr_t align_bits) {
  if (b != 4 && b != 8) return 0;
  return tok_nch(dtype, d, 32, align_bits);
}

}  // namespace stk
