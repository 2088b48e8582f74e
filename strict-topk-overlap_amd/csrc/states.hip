// Per-block softmax states, LSE merge, hybrid grouping, compact speculation
// and the touch_kv checksum.
//
// Reference kernels restated (6Mikao9/strict-topk-overlap):
//   strict_topk/kernels.py:42-71   _partial      -> k_states
//   strict_topk/gqa.py:29-59       _partial      -> k_states (GQA, slot mode)
//   strict_topk/kernels.py:74-91   _merge        -> k_merge
//   strict_topk/kernels.py:94-117  _group        -> k_hybrid_group1 (one round trip),
//                                                  k_hybrid_group (other shapes)
//   strict_topk/kernels.py:263-356 _mass_only / _compact_group / _compact_values
//   strict_topk/kernels.py:250-260 _touch        -> k_touch
#include "states_pack.hpp"
#include "api.hpp"

namespace stk {

// One wave per (query head, slot).  SLOT mode restates gqa.py:38-43: the slot
// is max{p : P[h,p] == A[h,s]} and only missing blocks are computed.
template <typename T, int VEC, int NC, int U, bool WITH_V, bool SLOT>
__global__ __launch_bounds__(256) void k_states(StatesArgs a) {
  const int waves = blockDim.x / STK_WAVE;
  int wg = a.remap ? xcd_remap(blockIdx.x, gridDim.x) : blockIdx.x;
  int64_t item = (int64_t)wg * waves + wave_id();
  int64_t items = (int64_t)a.hq * a.s;
  if (item >= items) return;
  int h = (int)(item / a.s);
  int j = (int)(item % a.s);
  int64_t row = item;
  int64_t bid = load_id(a.ids, a.itype, row);
  bool enabled = true;
  if (a.active_kind == 1) enabled = a.active[h] != 0;
  else if (a.active_kind == 2) enabled = a.active[row] != 0;
  if (SLOT) {
    int best = -1;
    for (int p = lane_id(); p < a.sp; p += STK_WAVE)
      if (load_id(a.pred, a.ptype, (int64_t)h * a.sp + p) == bid) best = p;
    for (int off = 1; off < STK_WAVE; off <<= 1) best = max(best, __shfl_xor(best, off));
    if (lane_id() == 0) a.slot[row] = best;
    enabled = best < 0;
  }
  if (a.slot_in && a.slot_in[(int64_t)(a.slot_shared ? 0 : h) * a.s + j] >= 0) return;
  if (bid < 0 || bid >= a.n) enabled = false;   // invalid IDs never touch memory
  Tile<T, VEC, NC> t;
  t.init(a.d);
  float m = -INFINITY, l = 0.f, acc[Tile<T, VEC, NC>::R];
#pragma unroll
  for (int i = 0; i < Tile<T, VEC, NC>::R; ++i) acc[i] = 0.f;
  if (enabled) {
    int g = a.hq / a.hkv;
    int kv = h / g;
    float qr[Tile<T, VEC, NC>::R];
    t.load_q(reinterpret_cast<const T*>(a.q) + (size_t)h * a.d, qr);
    size_t off = (((size_t)kv * a.n + (size_t)bid) * a.b) * a.d;
    const T* kb = reinterpret_cast<const T*>(a.k) + off;
    const T* vb = reinterpret_cast<const T*>(a.v) + off;
    float scale = 1.0f / sqrtf((float)a.d);
    t.template accum<U, false, WITH_V>(qr, kb, vb, a.b, scale, m, l, acc);
    t.finish(l, acc);
  } else if (SLOT) {
    return;   // hits keep their prediction state; scratch row left unwritten
  }
  if (lane_id() == 0) {
    a.m[row] = m;
    a.l[row] = l;
  }
  if (WITH_V) t.store(a.u + row * a.d, acc);
}

template <typename T, int NCH, int UP, typename I, bool ONE>
__global__ __launch_bounds__(256, NCH <= 4 ? 4 : 2) void k_states_tok(StatesArgs a) {
  states_tok_wg<T, NCH, UP, I, ONE>(a, a.remap ? xcd_remap(blockIdx.x, gridDim.x) : blockIdx.x);
}

// Small blocks (B = 4 or 8): one wave per (query head, 32-token pack).
template <typename T, int NCH, int BB, typename I>
__global__ __launch_bounds__(256, NCH <= 4 ? 4 : 2) void k_states_pack(StatesArgs a) {
  states_pack_wg<T, NCH, BB, I>(a, a.remap ? xcd_remap(blockIdx.x, gridDim.x) : blockIdx.x);
}

// Small blocks, HG query heads of a KV group per wave (one pack load when the
// heads' IDs agree at the pack).
template <typename T, int NCH, int BB, typename I, int HG>
__global__ __launch_bounds__(256, NCH <= 4 ? 4 : 2) void k_states_pack_grp(StatesArgs a) {
  states_pack_grp_wg<T, NCH, BB, I, HG>(a, a.remap ? xcd_remap(blockIdx.x, gridDim.x)
                                                   : blockIdx.x);
}

// The same with one merged state per pack (hierarchical exact and repair).
template <typename T, int NCH, int BB, typename I, int HG>
__global__ __launch_bounds__(256) void k_states_pack_comb(StatesArgs a) {
  states_pack_grp_wg<T, NCH, BB, I, HG, true>(a, a.remap ? xcd_remap(blockIdx.x, gridDim.x)
                                                         : blockIdx.x);
}

// LSE merge arguments (kernels.py:74-91, merge_partials :437-442).
struct MergeArgs {
  const float* m; const float* l; const float* u; const uint8_t* inc;
  int h, s, d;
  float* out;
};

// GQA states with one read of every (KV head, block) tile.  Wave (h, j)
// owns block b = ids[h, j] when no lower query head of its KV group lists b;
// the owner loads the K/V tile once and computes the state of every head of
// the group whose row holds b (writing each such slot), the other waves
// return.  Heads are processed in batches of HT sharing the loaded chunk.

template <typename T, int VEC, int NC, int U, typename I>
__global__ __launch_bounds__(256) void k_states_grp(StatesArgs a) {
  using TL = Tile<T, VEC, NC>;
  const int waves = blockDim.x / STK_WAVE;
  int wg = a.remap ? xcd_remap(blockIdx.x, gridDim.x) : blockIdx.x;
  int64_t item = (int64_t)wg * waves + wave_id();
  if (item >= (int64_t)a.hq * a.s) return;
  const I* ids = reinterpret_cast<const I*>(a.ids);
  const int h = (int)(item / a.s);
  const int G = a.hq / a.hkv;
  const int hl = h % G;
  const int g0 = h - hl;
  const int j = (int)(item - (int64_t)h * a.s);
  // rows of the group that list b (wave-uniform bit mask, G <= 64); the
  // group's G*S IDs are read 4 per lane at a time, all loads in flight.
  // When G*S <= 256 the wave's own ID comes out of the same registers.
  uint64_t found = 0ull;
  const int total = G * a.s;
  const I* grp = ids + (int64_t)g0 * a.s;
  int64_t bid;
  if (total <= 4 * STK_WAVE) {
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
    for (int i = 0; i < 4; ++i) {
      int x = i * STK_WAVE + lane_id();
      if (x < total && v[i] == bid) found |= 1ull << (x / a.s);
    }
  } else {
    bid = ids[item];
    for (int x0 = 0; x0 < total; x0 += 4 * STK_WAVE) {
      int64_t v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int x = x0 + i * STK_WAVE + lane_id();
        v[i] = ld_or(grp, (int64_t)x, x < total, (I)-1);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int x = x0 + i * STK_WAVE + lane_id();
        if (x < total && v[i] == bid) found |= 1ull << (x / a.s);
      }
    }
  }
  for (int off = 1; off < STK_WAVE; off <<= 1) found |= __shfl_xor(found, off);
  if (found & ((1ull << hl) - 1ull)) return;   // a lower head owns this block
  found &= ~((1ull << hl) - 1ull);
  const bool valid = bid >= 0 && bid < a.n;
  const int kv = h / G;
  TL t;
  t.init(a.d);
  const float scale = 1.0f / sqrtf((float)a.d);
  const size_t off = (((size_t)kv * a.n + (valid ? (size_t)bid : 0)) * a.b) * a.d;
  const T* kb = reinterpret_cast<const T*>(a.k) + off;
  const T* vb = reinterpret_cast<const T*>(a.v) + off;
  while (found) {
    int heads[kGrpHT];
    int nh = 0;
#pragma unroll
    for (int i = 0; i < kGrpHT; ++i) {
      heads[i] = hl;
      if (found) {
        int gg = __ffsll((long long)found) - 1;
        found &= found - 1;
        heads[i] = gg;
        nh = i + 1;
      }
    }
    float qr[kGrpHT][TL::R], m[kGrpHT], l[kGrpHT], acc[kGrpHT][TL::R];
    uint64_t pmask[kGrpHT];   // rows of at most 64 IDs: positions of b, read with q
#pragma unroll
    for (int i = 0; i < kGrpHT; ++i) {
      m[i] = -INFINITY;
      l[i] = 0.f;
#pragma unroll
      for (int r = 0; r < TL::R; ++r) acc[i][r] = 0.f;
      t.load_q(reinterpret_cast<const T*>(a.q) + (size_t)(g0 + heads[i]) * a.d, qr[i]);
      bool in = lane_id() < a.s;
      int64_t x = ld_or(ids, (int64_t)(g0 + heads[i]) * a.s + lane_id(), in, (I)-1);
      pmask[i] = __ballot(in && x == bid);
    }
    if (valid) {
      for (int t0 = 0; t0 < a.b; t0 += U * t.tpw) {
        Raw<T, VEC> kr[U][NC];
        Raw<T, VEC> vr[U][NC];
        t.template load_chunk<U, true>(kb, vb, t0, a.b, kr, vr);
#pragma unroll
        for (int i = 0; i < kGrpHT; ++i)
          if (i < nh)
            t.template update_chunk<U, false, true>(qr[i], kr, vr, t0, a.b, scale, m[i], l[i],
                                                    acc[i]);
      }
#pragma unroll
      for (int i = 0; i < kGrpHT; ++i)
        if (i < nh) t.finish(l[i], acc[i]);
    }
#pragma unroll
    for (int i = 0; i < kGrpHT; ++i) {
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

// LSE merge of S states per head in one pass over memory: every thread keeps
// an online (max, sum, vector) over the rows it reads, with all loads of a
// batch in flight, and the row groups are combined at the end.  Grid (heads,
// column tiles of 8 lanes * VEC dims); 32 row groups of 8 lanes.
template <int VEC>
__global__ __launch_bounds__(256) void k_merge2(MergeArgs a) {
  constexpr int LPR = 8, RG = 256 / LPR, RB = 4;
  __shared__ float part[RG][LPR * VEC];
  __shared__ float gm[RG], gz[RG];
  const int h = blockIdx.x;
  const int lc = threadIdx.x % LPR, rg = threadIdx.x / LPR;
  const int col = blockIdx.y * LPR * VEC + lc * VEC;
  const float* m = a.m + (size_t)h * a.s;
  const float* l = a.l + (size_t)h * a.s;
  const uint8_t* inc = a.inc ? a.inc + (size_t)h * a.s : nullptr;
  float mt = -INFINITY, zt = 0.f, acc[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) acc[v] = 0.f;
  for (int j0 = rg; j0 < a.s; j0 += RG * RB) {
    float mm[RB], ll[RB], uu[RB][VEC];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      int j = j0 + i * RG;
      bool in = j < a.s;
      bool on = in && (!inc || ld_or(inc, (int64_t)j, in, (uint8_t)0));
      float mv = ld_or(m, (int64_t)j, in, -INFINITY);
      float lv = ld_or(l, (int64_t)j, in, 0.f);
      const float* ur = a.u + ((size_t)h * a.s + (in ? j : 0)) * a.d;
      if constexpr (VEC == 4) {
        float4 x = *reinterpret_cast<const float4*>(ur + (col < a.d ? col : 0));
        uu[i][0] = x.x; uu[i][1] = x.y; uu[i][2] = x.z; uu[i][3] = x.w;
      } else {
        uu[i][0] = ur[col < a.d ? col : 0];
      }
      mm[i] = on ? mv : -INFINITY;
      ll[i] = on ? lv : 0.f;
#pragma unroll
      for (int v = 0; v < VEC; ++v) uu[i][v] = on ? uu[i][v] : 0.f;
    }
    float bm = mm[0];
#pragma unroll
    for (int i = 1; i < RB; ++i) bm = fmaxf(bm, mm[i]);
    float nm = fmaxf(mt, bm);
    float alpha = wexp(mt, nm);
    zt *= alpha;
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] *= alpha;
    mt = nm;
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      float w = wexp(mm[i], mt);
      zt += w * ll[i];
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] += w * uu[i][v];
    }
  }
#pragma unroll
  for (int v = 0; v < VEC; ++v) part[rg][lc * VEC + v] = acc[v];
  if (lc == 0) {
    gm[rg] = mt;
    gz[rg] = zt;
  }
  __syncthreads();
  if (rg == 0) {
    // reference frame: the max over included states, 0 when there is none
    float M = -INFINITY;
    for (int r = 0; r < RG; ++r) M = fmaxf(M, gm[r]);
    if (M == -INFINITY) M = 0.f;
    float zz = 0.f, f[RG];
    for (int r = 0; r < RG; ++r) {
      f[r] = wexp(gm[r], M);
      zz += f[r] * gz[r];
    }
    float inv = 1.f / fmaxf(zz, 1e-30f);
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      float sum = 0.f;
      for (int r = 0; r < RG; ++r) sum += f[r] * part[r][lc * VEC + v];
      if (col + v < a.d) a.out[(size_t)h * a.d + col + v] = sum * inv;
    }
  }
}

// Hybrid grouping (kernels.py:94-117).
struct GroupArgs {
  const float* m; const float* l; const float* u;
  int h, s, d; float tau;
  uint8_t* high; float* lm; float* ll; float* lu; float* labs;
};

__global__ __launch_bounds__(256) void k_hybrid_group(GroupArgs a) {
  __shared__ float red[32];
  __shared__ float part[2][256 * 4];
  int h = blockIdx.x;
  const float* m = a.m + (size_t)h * a.s;
  const float* l = a.l + (size_t)h * a.s;
  float gm = -INFINITY;
  for (int j = threadIdx.x; j < a.s; j += blockDim.x) gm = fmaxf(gm, m[j]);
  gm = block_max(gm, red);
  float tot = 0.f;
  for (int j = threadIdx.x; j < a.s; j += blockDim.x) tot += wexp(m[j], gm) * l[j];
  tot = block_sum(tot, red);
  float thr = a.tau * tot;
  float lmx = -INFINITY;
  for (int j = threadIdx.x; j < a.s; j += blockDim.x) {
    bool hi = wexp(m[j], gm) * l[j] >= thr;
    a.high[(size_t)h * a.s + j] = hi;
    if (!hi) lmx = fmaxf(lmx, m[j]);
  }
  lmx = block_max(lmx, red);
  if (lmx == -INFINITY) lmx = 0.f;
  int dt = 1;
  while (dt < a.d && dt < 256) dt <<= 1;
  int rg = 256 / dt;
  int tr = threadIdx.x / dt, td = threadIdx.x % dt;
  float acc[4] = {0.f, 0.f, 0.f, 0.f}, aab[4] = {0.f, 0.f, 0.f, 0.f};
  float z = 0.f;
  for (int j = tr; j < a.s; j += rg) {
    bool hi = wexp(m[j], gm) * l[j] >= thr;
    if (hi) continue;
    float w = wexp(m[j], lmx);
    if (td == 0) z += w * l[j];
    const float* ur = a.u + ((size_t)h * a.s + j) * a.d;
    for (int c = 0; c < 4; ++c) {
      int dd = td + c * dt;
      if (dd < a.d) {
        float x = ur[dd];
        acc[c] += w * x;
        aab[c] += w * fabsf(x);
      }
    }
  }
  z = block_sum(z, red);
  for (int c = 0; c < 4; ++c) {
    part[0][c * 256 + threadIdx.x] = acc[c];
    part[1][c * 256 + threadIdx.x] = aab[c];
  }
  __syncthreads();
  if (tr == 0) {
    for (int c = 0; c < 4; ++c) {
      int dd = td + c * dt;
      if (dd >= a.d) break;
      float s0 = 0.f, s1 = 0.f;
      for (int r = 0; r < rg; ++r) {
        s0 += part[0][c * 256 + r * dt + td];
        s1 += part[1][c * 256 + r * dt + td];
      }
      a.lu[(size_t)h * a.d + dd] = s0;
      a.labs[(size_t)h * a.d + dd] = s1;
    }
  }
  if (threadIdx.x == 0) {
    a.lm[h] = lmx;
    a.ll[h] = z;
  }
}

// The same grouping in one memory round trip, for S <= 256 state rows, D a
// multiple of 4 (<= 1024) and 16-byte aligned rows: every thread issues its
// m, l and the u rows it will weight at once; the row scalars pass through
// LDS once, after which every wave forms the same global max, total mass,
// high flags and low frame with wave reductions (no further barrier); the
// low aggregate and its envelope are summed per (row group, column) and
// folded through LDS.
constexpr int kGroupRows = 256;
constexpr int kGroupPF = 8;   // u float4s in flight per thread per pass

__device__ __forceinline__ bool group_high(float m, float l, float gm, float thr) {
  return wexp(m, gm) * l >= thr;
}

__global__ __launch_bounds__(256) void k_hybrid_group1(GroupArgs a) {
  __shared__ float s_m[kGroupRows], s_l[kGroupRows];
  __shared__ float4 s_pu[256], s_pa[256];
  const int h = blockIdx.x, tid = threadIdx.x, s = a.s, d = a.d;
  const float* M = a.m + (size_t)h * s;
  const float* L = a.l + (size_t)h * s;
  const float* U = a.u + (size_t)h * s * d;
  const float mv = tid < s ? M[tid] : -INFINITY;
  const float lv = tid < s ? L[tid] : 0.f;
  const int tpr = d >> 2, rgn = 256 / tpr;
  const int c4 = tid % tpr, rg = tid / tpr;
  const bool act = rg < rgn;
  const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 uu[kGroupPF];
  // every load is issued, rows past s (or idle threads) reading row 0 and
  // taking zeros: a load under a condition makes the compiler keep the
  // array in scratch memory
  auto fetch = [&](int pass) {
#pragma unroll
    for (int j = 0; j < kGroupPF; ++j) {
      const int r = rg + rgn * (pass * kGroupPF + j);
      const bool live = act && r < s;
      const float4 x = *reinterpret_cast<const float4*>(U + (size_t)(live ? r : 0) * d +
                                                        4 * (act ? c4 : 0));
      uu[j] = live ? x : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  fetch(0);
  s_m[tid] = mv;
  s_l[tid] = lv;
  __syncthreads();
  // ---- slot reductions, the same in every wave (lane l: rows l + 64 c)
  float pm[4], pl[4];
  float gm = -INFINITY;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int p = c * STK_WAVE + lane_id();
    pm[c] = p < s ? s_m[p] : -INFINITY;
    pl[c] = p < s ? s_l[p] : 0.f;
    gm = fmaxf(gm, pm[c]);
  }
  gm = wave_max_u(gm);
  float tot = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) tot += wexp(pm[c], gm) * pl[c];
  const float thr = a.tau * wave_sum_u(tot);
  bool hi[4];
  float lm = -INFINITY;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const bool ok = c * STK_WAVE + lane_id() < s;
    hi[c] = ok && group_high(pm[c], pl[c], gm, thr);
    lm = ok && !hi[c] ? fmaxf(lm, pm[c]) : lm;
  }
  lm = wave_max_u(lm);
  const float lowm = lm == -INFINITY ? 0.f : lm;
  float z = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const bool ok = c * STK_WAVE + lane_id() < s;
    z += ok && !hi[c] ? wexp(pm[c], lowm) * pl[c] : 0.f;
  }
  z = wave_sum_u(z);
  if (wave_id() == 0) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int p = c * STK_WAVE + lane_id();
      if (p < s) a.high[(size_t)h * s + p] = hi[c];
    }
    if (lane_id() == 0) {
      a.lm[h] = lowm;
      a.ll[h] = z;
    }
  }
  // ---- low aggregate and envelope of this thread's rows
  float4 lu = zero, la = zero;
  const int passes = (s + rgn * kGroupPF - 1) / (rgn * kGroupPF);
  for (int pass = 0; pass < passes; ++pass) {
    if (pass) fetch(pass);
#pragma unroll
    for (int j = 0; j < kGroupPF; ++j) {
      const int r = rg + rgn * (pass * kGroupPF + j);
      if (act && r < s) {
        const float mr = s_m[r], lr = s_l[r];
        const float wt = group_high(mr, lr, gm, thr) ? 0.f : wexp(mr, lowm);
        const float4 x = uu[j];
        lu.x += wt * x.x; lu.y += wt * x.y; lu.z += wt * x.z; lu.w += wt * x.w;
        la.x += wt * fabsf(x.x); la.y += wt * fabsf(x.y);
        la.z += wt * fabsf(x.z); la.w += wt * fabsf(x.w);
      }
    }
  }
  s_pu[tid] = lu;
  s_pa[tid] = la;
  __syncthreads();
  if (tid < tpr) {
    float4 su = zero, sa = zero;
    for (int g = 0; g < rgn; ++g) {
      const float4 x = s_pu[g * tpr + tid], y = s_pa[g * tpr + tid];
      su.x += x.x; su.y += x.y; su.z += x.z; su.w += x.w;
      sa.x += y.x; sa.y += y.y; sa.z += y.z; sa.w += y.w;
    }
    *reinterpret_cast<float4*>(a.lu + (size_t)h * d + 4 * tid) = su;
    *reinterpret_cast<float4*>(a.labs + (size_t)h * d + 4 * tid) = sa;
  }
}

static bool group1_covers(int s, int d, const float* u, const float* lu, const float* labs) {
  const uintptr_t bits = reinterpret_cast<uintptr_t>(u) | reinterpret_cast<uintptr_t>(lu) |
                         reinterpret_cast<uintptr_t>(labs);
  return s <= kGroupRows && d % 4 == 0 && d <= 1024 && (bits & 15) == 0;
}

// Compact grouping (kernels.py:281-309): rank high blocks in position order,
// cap at C, overflow flag, retained IDs padded with -1, low (m, l).
struct CompactArgs {
  const void* q; const void* k; const void* v;
  const void* ids; int itype;
  int hq, hkv, n, b, d, s, c;
  float tau;
  const float* pm; const float* pl;
  uint8_t* high; void* rids; uint8_t* overflow;
  float* lm; float* ll; float* lu; float* labs;
  float* m; float* l; float* u;
};

constexpr int kCompactMaxS = 32768;

__global__ __launch_bounds__(256) void k_compact_group(CompactArgs a) {
  __shared__ float red[32];
  __shared__ int scan[256];
  __shared__ uint32_t lowbits[kCompactMaxS / 32];
  int h = blockIdx.x;
  const float* m = a.pm + (size_t)h * a.s;
  const float* l = a.pl + (size_t)h * a.s;
  float gm = -INFINITY;
  for (int j = threadIdx.x; j < a.s; j += blockDim.x) gm = fmaxf(gm, m[j]);
  gm = block_max(gm, red);
  float tot = 0.f;
  for (int j = threadIdx.x; j < a.s; j += blockDim.x) tot += wexp(m[j], gm) * l[j];
  tot = block_sum(tot, red);
  float thr = a.tau * tot;
  for (int j = threadIdx.x; j < a.c; j += blockDim.x)
    store_id(a.rids, a.itype, (int64_t)h * a.c + j, -1);
  for (int j = threadIdx.x; j < (a.s + 31) / 32; j += blockDim.x) lowbits[j] = 0u;
  __syncthreads();
  // rank = inclusive prefix count of high blocks in position order
  int carry = 0;
  float lmx = -INFINITY;
  for (int j0 = 0; j0 < a.s; j0 += blockDim.x) {
    int j = j0 + threadIdx.x;
    int hi = (j < a.s) && (wexp(m[j], gm) * l[j] >= thr);
    scan[threadIdx.x] = hi;
    __syncthreads();
    for (int off = 1; off < (int)blockDim.x; off <<= 1) {
      int x = (int)threadIdx.x >= off ? scan[threadIdx.x - off] : 0;
      __syncthreads();
      scan[threadIdx.x] += x;
      __syncthreads();
    }
    int rank = carry + scan[threadIdx.x];
    int total = scan[blockDim.x - 1];
    __syncthreads();
    if (j < a.s) {
      bool keep = hi && rank <= a.c;
      a.high[(size_t)h * a.s + j] = keep;
      if (keep) {
        store_id(a.rids, a.itype, (int64_t)h * a.c + rank - 1,
                 load_id(a.ids, a.itype, (int64_t)h * a.s + j));
      } else {
        lmx = fmaxf(lmx, m[j]);
        atomicOr(&lowbits[j >> 5], 1u << (j & 31));
      }
    }
    carry += total;
  }
  lmx = block_max(lmx, red);
  if (lmx == -INFINITY) lmx = 0.f;
  float z = 0.f;
  for (int j = threadIdx.x; j < a.s; j += blockDim.x)
    if ((lowbits[j >> 5] >> (j & 31)) & 1u) z += wexp(m[j], lmx) * l[j];
  z = block_sum(z, red);
  if (threadIdx.x == 0) {
    a.overflow[h] = carry > a.c;
    a.lm[h] = lmx;
    a.ll[h] = z;
  }
}

// Compact values (kernels.py:312-356): workgroup slot 0 walks the low blocks
// of head h in the low frame (per token, with the abs envelope); slots 1..C
// compute retained block states.  Low blocks are split over the 4 waves and
// the wave sums are added in wave order.
template <typename T, int VEC, int NC, int U>
__global__ __launch_bounds__(256) void k_compact_values(CompactArgs a) {
  using TL = Tile<T, VEC, NC>;
  __shared__ float wl[4];
  __shared__ float wu[2][4][kMaxD];
  int h = blockIdx.x;
  int slot = blockIdx.y;
  int g = a.hq / a.hkv;
  int kv = h / g;
  TL t;
  t.init(a.d);
  float qr[TL::R];
  t.load_q(reinterpret_cast<const T*>(a.q) + (size_t)h * a.d, qr);
  float scale = 1.0f / sqrtf((float)a.d);
  const T* K = reinterpret_cast<const T*>(a.k);
  const T* V = reinterpret_cast<const T*>(a.v);
  if (slot == 0) {
    float lmx = a.lm[h];
    float l = 0.f, acc[TL::R], aab[TL::R];
#pragma unroll
    for (int i = 0; i < TL::R; ++i) acc[i] = aab[i] = 0.f;
    for (int j = wave_id(); j < a.s; j += 4) {
      if (a.high[(size_t)h * a.s + j]) continue;
      int64_t bid = load_id(a.ids, a.itype, (int64_t)h * a.s + j);
      if (bid < 0 || bid >= a.n) continue;
      size_t off = (((size_t)kv * a.n + bid) * a.b) * a.d;
      t.template accum_fixed_abs<U>(qr, K + off, V + off, a.b, scale, lmx, l, acc, aab);
    }
    t.finish(l, acc);
    float dummy = 0.f;
    t.finish(dummy, aab);
    if (t.tok == 0) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        int base = (t.part + c * t.lpt) * VEC;
#pragma unroll
        for (int i = 0; i < VEC; ++i)
          if (base + i < a.d) {
            wu[0][wave_id()][base + i] = acc[c * VEC + i];
            wu[1][wave_id()][base + i] = aab[c * VEC + i];
          }
      }
    }
    __syncthreads();
    for (int dd = threadIdx.x; dd < a.d; dd += blockDim.x) {
      float s0 = 0.f, s1 = 0.f;
      for (int w = 0; w < 4; ++w) {
        s0 += wu[0][w][dd];
        s1 += wu[1][w][dd];
      }
      a.lu[(size_t)h * a.d + dd] = s0;
      a.labs[(size_t)h * a.d + dd] = s1;
    }
    (void)wl;
    return;
  }
  // retained slots: one wave per slot (waves 1..3 idle)
  if (wave_id() != 0) return;
  int c = slot - 1;
  int64_t row = (int64_t)h * a.c + c;
  int64_t bid = load_id(a.rids, a.itype, row);
  float m = -INFINITY, l = 0.f, acc[TL::R];
#pragma unroll
  for (int i = 0; i < TL::R; ++i) acc[i] = 0.f;
  if (bid >= 0 && bid < a.n) {
    size_t off = (((size_t)kv * a.n + bid) * a.b) * a.d;
    t.template accum<U, false, true>(qr, K + off, V + off, a.b, scale, m, l, acc);
    t.finish(l, acc);
  }
  if (lane_id() == 0) {
    a.m[row] = m;
    a.l[row] = l;
  }
  t.store(a.u + row * a.d, acc);
}

// touch_kv checksum (kernels.py:250-260): one wave per (head, slot, tile).
template <typename T>
__global__ __launch_bounds__(64) void k_touch(const T* k, const T* v, const void* ids, int itype,
                                              int h, int n, int b, int d, int s, float* out) {
  int hh = blockIdx.x, j = blockIdx.y, tile = blockIdx.z;
  int ntiles = gridDim.z;
  int64_t bid = load_id(ids, itype, (int64_t)hh * s + j);
  float sum = 0.f;
  if (bid >= 0 && bid < n) {
    size_t base = ((size_t)hh * n + bid) * (size_t)b * d;
    for (int x = tile * 1024 + threadIdx.x; x < min((tile + 1) * 1024, b * d); x += 64)
      sum += cvt(k[base + x]) + cvt(v[base + x]);
  }
  sum = wave_sum(sum);
  if (threadIdx.x == 0) out[((size_t)hh * s + j) * ntiles + tile] = sum;
}

}  // namespace stk

using namespace stk;

// ---------------------------------------------------------------- C ABI
static int launch_states(StatesArgs& a, int dtype, bool with_v, bool slot, hipStream_t st) {
  int64_t items = (int64_t)a.hq * a.s;
  if (items == 0) return STK_OK;
  int grid = (int)((items + 3) / 4);
  a.remap = grid >= 8 ? 1 : 0;
  const int G = a.hq / a.hkv;
  const uintptr_t align = reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.k) |
                          reinterpret_cast<uintptr_t>(a.v);
  const int pnch = with_v && !slot ? pack_nch(dtype, a.d, a.b, align) : 0;
  if (pnch && !a.slot_in && a.active_kind == 0 &&
      stk_hier_mfma_covers(dtype, a.hq, a.hkv, a.b, a.d,
                           align | reinterpret_cast<uintptr_t>(a.u))) {
    // 8-16 query heads per KV head: the group's block states on the matrix
    // cores (hier_mfma.hip)
    return stk_launch_hier_mfma(a.q, a.k, a.v, dtype, a.hq, a.hkv, a.n, a.b, a.d, a.ids, a.itype,
                                a.s, a.m, a.l, a.u, 1, st);
  }
  if (pnch) {
    const int64_t packs = (int64_t)a.hq * ((a.s + 32 / a.b - 1) / (32 / a.b));
    const int pgrid = (int)((packs + 3) / 4);
    a.remap = pgrid >= 8 ? 1 : 0;
    const bool i64 = a.itype == IT_I64;
    // GQA: four (or two) heads of a KV group per wave
    const int hg = G % 4 == 0 ? 4 : (G % 2 == 0 ? 2 : 1);
    if (hg > 1) {
      const int ggrid = (int)((packs / hg + 3) / 4);
      a.remap = ggrid >= 8 ? 1 : 0;
#define STK_PACKG(BBV, HGV)                                                                        \
      STK_DISPATCH_TOK(dtype, pnch, {                                                              \
        if (i64)                                                                                   \
          hipLaunchKernelGGL((k_states_pack_grp<T, NCH, BBV, int64_t, HGV>), dim3(ggrid), dim3(256), \
                             0, st, a);                                                            \
        else                                                                                       \
          hipLaunchKernelGGL((k_states_pack_grp<T, NCH, BBV, int32_t, HGV>), dim3(ggrid), dim3(256), \
                             0, st, a);                                                            \
      })
      if (a.b == 4 && hg == 4) STK_PACKG(4, 4);
      else if (a.b == 4) STK_PACKG(4, 2);
      else if (hg == 4) STK_PACKG(8, 4);
      else STK_PACKG(8, 2);
#undef STK_PACKG
      return stk_check_launch("k_states_pack_grp");
    }
#define STK_PACK(BBV)                                                                              \
    STK_DISPATCH_TOK(dtype, pnch, {                                                                \
      if (i64)                                                                                     \
        hipLaunchKernelGGL((k_states_pack<T, NCH, BBV, int64_t>), dim3(pgrid), dim3(256), 0, st, a); \
      else                                                                                         \
        hipLaunchKernelGGL((k_states_pack<T, NCH, BBV, int32_t>), dim3(pgrid), dim3(256), 0, st, a); \
    })
    if (a.b == 4) STK_PACK(4);
    else STK_PACK(8);
#undef STK_PACK
    return stk_check_launch("k_states_pack");
  }
  const int nch = with_v && !slot && !a.slot_in ? tok_nch(dtype, a.d, a.b, align) : 0;
  if (nch) {
    const bool i64 = a.itype == IT_I64;
    const bool one = tok_up(a.b) == 1;
#define STK_TOK(UPV, ONE)                                                                       \
    STK_DISPATCH_TOK(dtype, nch, {                                                              \
      if (i64)                                                                                  \
        hipLaunchKernelGGL((k_states_tok<T, NCH, UPV, int64_t, ONE>), dim3(grid), dim3(256), 0, st, a); \
      else                                                                                      \
        hipLaunchKernelGGL((k_states_tok<T, NCH, UPV, int32_t, ONE>), dim3(grid), dim3(256), 0, st, a); \
    })
    if (a.b == 16) STK_TOK(1, true);     // whole block in one chunk
    else if (one) STK_TOK(1, false);
    else if (a.b == 32) STK_TOK(2, true);
    else STK_TOK(2, false);
#undef STK_TOK
    return stk_check_launch("k_states_tok");
  }
  const bool dedupe = with_v && !slot && !a.active && !a.slot_in && G > 1 && G <= 64 &&
                      (int64_t)G * a.s <= 4096;
  STK_DISPATCH_TILE(dtype, a.d, {
    if (dedupe && a.itype == IT_I64)
      hipLaunchKernelGGL((k_states_grp<T, VEC, NC, U, int64_t>), dim3(grid), dim3(256), 0, st, a);
    else if (dedupe)
      hipLaunchKernelGGL((k_states_grp<T, VEC, NC, U, int32_t>), dim3(grid), dim3(256), 0, st, a);
    else if (slot)
      hipLaunchKernelGGL((k_states<T, VEC, NC, U, true, true>), dim3(grid), dim3(256), 0, st, a);
    else if (with_v)
      hipLaunchKernelGGL((k_states<T, VEC, NC, U, true, false>), dim3(grid), dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((k_states<T, VEC, NC, U, false, false>), dim3(grid), dim3(256), 0, st, a);
  });
  return stk_check_launch("k_states");
}

int stk_launch_states(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                      int n, int b, int d, const void* ids, int itype, int s,
                      const uint8_t* active, int active_kind, const void* pred, int ptype, int sp,
                      int32_t* slot, float* m, float* l, float* u, bool with_v, hipStream_t st) {
  StatesArgs a{};
  a.q = q; a.k = k; a.v = v; a.ids = ids; a.itype = itype;
  a.hq = hq; a.hkv = hkv; a.n = n; a.b = b; a.d = d; a.s = s;
  a.active = active; a.active_kind = active ? active_kind : 0;
  a.pred = pred; a.ptype = ptype; a.sp = sp; a.slot = slot;
  a.m = m; a.l = l; a.u = u;
  return launch_states(a, dtype, with_v, slot != nullptr, st);
}

int stk_launch_states_skip(const void* q, const void* k, const void* v, int dtype, int hq,
                           int hkv, int n, int b, int d, const void* ids, int itype, int s,
                           const int32_t* slot_in, int slot_shared, float* m, float* l, float* u,
                           hipStream_t st) {
  StatesArgs a{};
  a.q = q; a.k = k; a.v = v; a.ids = ids; a.itype = itype;
  a.hq = hq; a.hkv = hkv; a.n = n; a.b = b; a.d = d; a.s = s;
  a.m = m; a.l = l; a.u = u;
  a.slot_in = slot_in; a.slot_shared = slot_shared;
  return launch_states(a, dtype, true, false, st);
}

bool stk_states_comb_covers(int dtype, int hq, int hkv, int b, int d, uintptr_t align) {
  const int G = hq / hkv;
  return pack_nch(dtype, d, b, align) != 0 && G % 2 == 0;
}

int stk_launch_states_comb(const void* q, const void* k, const void* v, int dtype, int hq,
                           int hkv, int n, int b, int d, const void* ids, int itype, int s,
                           const int32_t* slot_in, int slot_shared, const float* pm,
                           const float* pl, const float* pu, int psp, float* m, float* l,
                           float* u, hipStream_t st) {
  StatesArgs a{};
  a.q = q; a.k = k; a.v = v; a.ids = ids; a.itype = itype;
  a.hq = hq; a.hkv = hkv; a.n = n; a.b = b; a.d = d; a.s = s;
  a.m = m; a.l = l; a.u = u;
  a.slot_in = slot_in; a.slot_shared = slot_shared;
  a.combine = 1; a.pm = pm; a.pl = pl; a.pu = pu; a.psp = psp;
  const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(v);
  const int pnch = pack_nch(dtype, d, b, align);
  const int G = hq / hkv;
  if (!pnch || G % 2 != 0 || s <= 0) return STK_EINVAL;
  if (slot_in && (!pm || !pl || !pu || psp <= 0)) return STK_EINVAL;
  const int hg = G % 4 == 0 ? 4 : 2;
  // one workgroup per (KV head, four packs, head group)
  const int pgroups = ((s + 32 / b - 1) / (32 / b) + 3) / 4;
  const int grid = hkv * pgroups * (G / hg);
  a.remap = grid >= 8 ? 1 : 0;
  const bool i64 = itype == IT_I64;
#define STK_COMB(BBV, HGV)                                                                        \
  STK_DISPATCH_TOK(dtype, pnch, {                                                                 \
    if (i64)                                                                                      \
      hipLaunchKernelGGL((k_states_pack_comb<T, NCH, BBV, int64_t, HGV>), dim3(grid), dim3(256),  \
                         0, st, a);                                                               \
    else                                                                                          \
      hipLaunchKernelGGL((k_states_pack_comb<T, NCH, BBV, int32_t, HGV>), dim3(grid), dim3(256),  \
                         0, st, a);                                                               \
  })
  if (b == 4 && hg == 4) STK_COMB(4, 4);
  else if (b == 4) STK_COMB(4, 2);
  else if (hg == 4) STK_COMB(8, 4);
  else STK_COMB(8, 2);
#undef STK_COMB
  return stk_check_launch("k_states_pack_comb");
}

int stk_launch_merge(const float* m, const float* l, const float* u, const uint8_t* inc, int h,
                     int s, int d, float* out, hipStream_t st) {
  MergeArgs a{m, l, u, inc, h, s, d, out};
  // vector path needs 16-byte aligned rows (d % 4 == 0 and an aligned base)
  bool vec = d % 4 == 0 && (reinterpret_cast<uintptr_t>(u) & 15) == 0;
  if (vec)
    hipLaunchKernelGGL(k_merge2<4>, dim3(h, (d + 31) / 32), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(k_merge2<1>, dim3(h, (d + 7) / 8), dim3(256), 0, st, a);
  return stk_check_launch("k_merge");
}

extern "C" {

STK_API int stk_block_partials(const void* q, const void* k, const void* v, int dtype, int hq,
                               int hkv, int n, int b, int d, const void* ids, int id_dtype, int s,
                               const uint8_t* active, int active_kind, float* m, float* l, float* u,
                               void* stream) {
  STK_REQUIRE(stk_check_kv(dtype, hq, hkv, n, b, d));
  STK_REQUIRE(q && k && v && ids && m && l && u, "null pointer");
  STK_REQUIRE(s >= 0 && (id_dtype == IT_I32 || id_dtype == IT_I64), "bad ids");
  STK_REQUIRE(active_kind >= 0 && active_kind <= 2, "bad active kind");
  return stk_launch_states(q, k, v, dtype, hq, hkv, n, b, d, ids, id_dtype, s, active, active_kind,
                           nullptr, 0, 0, nullptr, m, l, u, true, (hipStream_t)stream);
}

STK_API int stk_merge_partials(const float* m, const float* l, const float* u,
                               const uint8_t* include, int h, int s, int d, float* out,
                               void* stream) {
  STK_REQUIRE(m && l && u && out, "null pointer");
  STK_REQUIRE(h >= 0 && s > 0 && d > 0 && d <= kMaxD, "bad merge shape");
  if (h == 0) return STK_OK;
  return stk_launch_merge(m, l, u, include, h, s, d, out, (hipStream_t)stream);
}

STK_API size_t stk_exact_workspace_bytes(int hq, int s, int d) {
  return stk_align((size_t)hq * s * 4) * 2 + stk_align((size_t)hq * s * d * 4);
}

STK_API int stk_exact_attention(const void* q, const void* k, const void* v, int dtype, int hq,
                                int hkv, int n, int b, int d, const void* ids, int id_dtype, int s,
                                float* out, void* workspace, size_t workspace_bytes,
                                void* stream) {
  STK_REQUIRE(stk_check_kv(dtype, hq, hkv, n, b, d));
  STK_REQUIRE(q && k && v && ids && out, "null pointer");
  STK_REQUIRE(s > 0, "ids must be nonempty");
  STK_REQUIRE(workspace && workspace_bytes >= stk_exact_workspace_bytes(hq, s, d),
              "workspace too small");
  Carve w(workspace);
  float* m = w.take<float>((size_t)hq * s);
  float* l = w.take<float>((size_t)hq * s);
  float* u = w.take<float>((size_t)hq * s * d);
  hipStream_t st = (hipStream_t)stream;
  int rc = stk_launch_states(q, k, v, dtype, hq, hkv, n, b, d, ids, id_dtype, s, nullptr, 0,
                             nullptr, 0, 0, nullptr, m, l, u, true, st);
  if (rc) return rc;
  return stk_launch_merge(m, l, u, nullptr, hq, s, d, out, st);
}

STK_API int stk_speculate(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                          int n, int b, int d, const void* pred, int pred_dtype, int s, int mode,
                          float tau, int capacity, float* m, float* l, float* u, uint8_t* high,
                          float* low_m, float* low_l, float* low_u, float* low_abs,
                          void* retained_ids, uint8_t* overflow, float* mass_m, float* mass_l,
                          void* stream) {
  STK_REQUIRE(stk_check_kv(dtype, hq, hkv, n, b, d));
  STK_REQUIRE(q && k && v && pred && m && l && u, "null pointer");
  STK_REQUIRE(s > 0, "predicted ids must be nonempty");
  STK_REQUIRE(mode >= 0 && mode <= 2, "mode must be 0 (saved), 1 (hybrid) or 2 (compact)");
  STK_REQUIRE(tau >= 0.f && tau <= 1.f, "mass_threshold must be in [0,1]");
  hipStream_t st = (hipStream_t)stream;
  if (mode != 2) {
    int rc = stk_launch_states(q, k, v, dtype, hq, hkv, n, b, d, pred, pred_dtype, s, nullptr, 0,
                               nullptr, 0, 0, nullptr, m, l, u, true, st);
    if (rc || mode == 0) return rc;
    STK_REQUIRE(high && low_m && low_l && low_u && low_abs, "null hybrid output");
    GroupArgs g{m, l, u, hq, s, d, tau, high, low_m, low_l, low_u, low_abs};
    if (group1_covers(s, d, u, low_u, low_abs)) {
      hipLaunchKernelGGL(k_hybrid_group1, dim3(hq), dim3(256), 0, st, g);
      return stk_check_launch("k_hybrid_group1");
    }
    hipLaunchKernelGGL(k_hybrid_group, dim3(hq), dim3(256), 0, st, g);
    return stk_check_launch("k_hybrid_group");
  }
  STK_REQUIRE(high && low_m && low_l && low_u && low_abs && retained_ids && overflow && mass_m &&
                  mass_l,
              "null compact output");
  STK_REQUIRE(capacity >= 1 && capacity <= s, "bad compact capacity");
  STK_REQUIRE(s <= kCompactMaxS, "compact speculation supports at most 32768 predicted blocks");
  int rc = stk_launch_states(q, k, v, dtype, hq, hkv, n, b, d, pred, pred_dtype, s, nullptr, 0,
                             nullptr, 0, 0, nullptr, mass_m, mass_l, nullptr, false, st);
  if (rc) return rc;
  CompactArgs c{};
  c.q = q; c.k = k; c.v = v; c.ids = pred; c.itype = pred_dtype;
  c.hq = hq; c.hkv = hkv; c.n = n; c.b = b; c.d = d; c.s = s; c.c = capacity; c.tau = tau;
  c.pm = mass_m; c.pl = mass_l; c.high = high; c.rids = retained_ids; c.overflow = overflow;
  c.lm = low_m; c.ll = low_l; c.lu = low_u; c.labs = low_abs; c.m = m; c.l = l; c.u = u;
  hipLaunchKernelGGL(k_compact_group, dim3(hq), dim3(256), 0, st, c);
  rc = stk_check_launch("k_compact_group");
  if (rc) return rc;
  STK_DISPATCH_TILE(dtype, d, {
    hipLaunchKernelGGL((k_compact_values<T, VEC, NC, U>), dim3(hq, capacity + 1), dim3(256), 0,
                       st, c);
  });
  return stk_check_launch("k_compact_values");
}

STK_API int stk_touch_kv(const void* k, const void* v, int dtype, int h, int n, int b, int d,
                         const void* pred, int pred_dtype, int s, float* out, void* stream) {
  STK_REQUIRE(stk_check_kv(dtype, h, h, n, b, d));
  STK_REQUIRE(k && v && pred && out, "null pointer");
  if (s == 0 || h == 0) return STK_OK;
  int nt = (b * d + 1023) / 1024;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DT_BF16)
    hipLaunchKernelGGL(k_touch<bf16s>, dim3(h, s, nt), dim3(64), 0, st, (const bf16s*)k,
                       (const bf16s*)v, pred, pred_dtype, h, n, b, d, s, out);
  else if (dtype == DT_F16)
    hipLaunchKernelGGL(k_touch<f16s>, dim3(h, s, nt), dim3(64), 0, st, (const f16s*)k,
                       (const f16s*)v, pred, pred_dtype, h, n, b, d, s, out);
  else
    hipLaunchKernelGGL(k_touch<float>, dim3(h, s, nt), dim3(64), 0, st, (const float*)k,
                       (const float*)v, pred, pred_dtype, h, n, b, d, s, out);
  return stk_check_launch("k_touch");
}

}  // extern "C"
