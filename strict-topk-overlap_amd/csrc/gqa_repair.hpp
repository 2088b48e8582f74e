// Single-workgroup saved / union repair of one query head for native GQA.
#pragma once

#include "head.hpp"
#include "tile2.hpp"

namespace stk {

// ------------------------------------------------------------ native GQA
// One 512-thread workgroup per query head does the whole saved / union
// repair (strict_topk/gqa.py:164-193, gqa_light.py:10-92):
//   1. slot[a] = max{p : P[p] == A[a]} through an LDS map over block IDs
//      (N <= kRepairMapN; brute force over P in LDS otherwise), and the hit
//      rows and missed blocks compacted in position order;
//   2. A-waves merge the reused prediction states (the hits, or every
//      predicted state in union mode) with an online softmax over batches of
//      rows whose loads are all in flight, while B-waves concurrently stream
//      the missed blocks' K/V tiles (the next tile's loads issued before the
//      current tile's arithmetic);
//   3. one LSE merge of the per-wave states.
constexpr int kRepairThreads = 512;
constexpr int kRepairWaves = kRepairThreads / STK_WAVE;
constexpr int kRepairMapN = 8192;
constexpr int kRowLanes = 16;      // lanes per state row (8 columns each per 128-col chunk)

struct GqaRepairArgs {
  KV kv;
  const void* a; int atype; int sa;
  const void* p; int ptype; int sp;
  const float* pm; const float* pl; const float* pu;
  int uni;
  float* out;
};

// Membership of one head's rows, staged in LDS.  After the call:
//   ids[0 .. *nm)   missed block IDs (valid, absent from P), position order
//   rows[0 .. *nh)  slots of the hits, position order
// With staged, ids[0 .. SA) already holds the selected row.
__device__ __forceinline__ void repair_membership(const GqaRepairArgs& a, int h, int* map,
                                                  int* ids, int* rows, int* pids, int* tmp,
                                                  int* nh, int* nm, bool staged) {
  const int n = a.kv.n;
  const bool use_map = n <= kRepairMapN;
  // the predicted row's IDs are requested with the selected row's (up to
  // two per thread; longer rows load theirs after the map is cleared)
  const bool pre = use_map && a.sp <= 2 * (int)blockDim.x;
  int64_t pv[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int p = threadIdx.x + r * (int)blockDim.x;
    pv[r] = pre && p < a.sp ? load_id(a.p, a.ptype, (int64_t)h * a.sp + p) : -1;
  }
  if (use_map)
    for (int i = threadIdx.x; i < n; i += blockDim.x) map[i] = 0;
  if (!staged)
    for (int j = threadIdx.x; j < a.sa; j += blockDim.x)
      ids[j] = (int)load_id(a.a, a.atype, (int64_t)h * a.sa + j);
  if (!use_map)
    for (int p = threadIdx.x; p < a.sp; p += blockDim.x)
      pids[p] = (int)load_id(a.p, a.ptype, (int64_t)h * a.sp + p);
  __syncthreads();
  if (use_map) {
    if (pre) {
#pragma unroll
      for (int r = 0; r < 2; ++r)
        if (pv[r] >= 0 && pv[r] < n) atomicMax(&map[pv[r]], threadIdx.x + r * (int)blockDim.x + 1);
    } else {
      for (int p = threadIdx.x; p < a.sp; p += blockDim.x) {
        int64_t id = load_id(a.p, a.ptype, (int64_t)h * a.sp + p);
        if (id >= 0 && id < n) atomicMax(&map[id], p + 1);
      }
    }
    __syncthreads();
  }
  // contiguous slice of A positions per thread, so scans keep position order
  const int per = (a.sa + (int)blockDim.x - 1) / (int)blockDim.x;   // <= 8
  const int j0 = threadIdx.x * per, j1 = min(a.sa, j0 + per);
  int my_id[8], my_slot[8];
  int nhit = 0, nmiss = 0;
  for (int j = j0, c = 0; j < j1; ++j, ++c) {
    int id = ids[j];
    int slot = -1;
    if (id >= 0 && id < n) {
      if (use_map) slot = map[id] - 1;
      else
        for (int p = 0; p < a.sp; ++p) slot = pids[p] == id ? p : slot;
    }
    my_id[c] = id;
    my_slot[c] = slot;
    nhit += slot >= 0;
    nmiss += slot < 0 && id >= 0 && id < n;
  }
  // one scan of packed counts (at most 8 positions per thread, so both
  // totals stay below 2^16)
  int total;
  const int pre_sum = block_excl_scan1(nhit | (nmiss << 16), tmp, &total);
  int hpos = pre_sum & 0xffff, mpos = pre_sum >> 16;
  const int total_hit = total & 0xffff, total_miss = total >> 16;
  for (int j = j0, c = 0; j < j1; ++j, ++c) {
    if (my_slot[c] >= 0) rows[hpos++] = my_slot[c];
    else if (my_id[c] >= 0 && my_id[c] < n) ids[mpos++] = my_id[c];   // compacted in place
  }
  *nh = total_hit;
  *nm = total_miss;
  __syncthreads();
}

// Streaming of a list of KV blocks (IDs in LDS, entries x0, x0 + stride, ...)
// through one wave with the online softmax; the next chunk's loads are
// issued before the arithmetic on the current one, without branches (past
// the last chunk the current one is read again).  The result (m, l) is
// returned and the D-vector written to out[].
template <typename T, int VEC, int NC, int U>
struct GenericStream {
  __device__ __forceinline__ static void run(const KV& kv_, int h, const int* list, int x0,
                                             int count, int stride, float& m, float& l,
                                             float* out) {
    using TL = Tile<T, VEC, NC>;
    const int d = kv_.d, n = kv_.n, B = kv_.b;
    TL t;
    t.init(d);
    float qr[TL::R];
    t.load_q(reinterpret_cast<const T*>(kv_.q) + (size_t)h * d, qr);
    const int kv = h / (kv_.hq / kv_.hkv);
    const float scale = 1.0f / sqrtf((float)d);
    const T* K = (const T*)kv_.k;
    const T* V = (const T*)kv_.v;
    float tacc[TL::R];
#pragma unroll
    for (int i = 0; i < TL::R; ++i) tacc[i] = 0.f;
    Raw<T, VEC> kr[U][NC], vr[U][NC];
    int x = x0;
    const int step = U * t.tpw;
    int cur_id = x < count ? list[x] : 0;
    {
      size_t off = (((size_t)kv * n + cur_id) * B) * d;
      t.template load_chunk<U, true>(K + off, V + off, 0, B, kr, vr);
    }
    for (int t0 = 0; x < count;) {
      int nt0 = t0 + step;
      int nx = x;
      if (nt0 >= B) {
        nt0 = 0;
        nx = x + stride;
      }
      const bool have_next = nx < count;
      const int nid = have_next ? list[nx] : cur_id;
      const int lt0 = have_next ? nt0 : t0;
      size_t noff = (((size_t)kv * n + nid) * B) * d;
      Raw<T, VEC> kn[U][NC], vn[U][NC];
      t.template load_chunk<U, true>(K + noff, V + noff, lt0, B, kn, vn);
      t.template update_chunk<U, false, true>(qr, kr, vr, t0, B, scale, m, l, tacc);
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          kr[u][c] = kn[u][c];
          vr[u][c] = vn[u][c];
        }
      x = nx;
      t0 = nt0;
      cur_id = nid;
    }
    t.finish(l, tacc);
    if (t.tok == 0) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        int base = (t.part + c * t.lpt) * VEC;
#pragma unroll
        for (int i = 0; i < VEC; ++i)
          if (base + i < d) out[base + i] = tacc[c * VEC + i];
      }
    }
  }
};

template <typename T, int NCH, int UP>
struct TokStream {
  __device__ __forceinline__ static void run(const KV& kv_, int h, const int* list, int x0,
                                             int count, int stride, float& m, float& l,
                                             float* out) {
    using TT = TokTile<T, NCH, UP>;
    const int d = kv_.d, n = kv_.n, B = kv_.b;
    TT t;
    t.init();
    uint32_t qw[TT::QW];
    t.load_q(reinterpret_cast<const T*>(kv_.q) + (size_t)h * d, qw);
    const int kv = h / (kv_.hq / kv_.hkv);
    const float scale = 1.0f / sqrtf((float)d);
    const T* K = (const T*)kv_.k;
    const T* V = (const T*)kv_.v;
    float acc[TT::DPL];
#pragma unroll
    for (int e = 0; e < TT::DPL; ++e) acc[e] = 0.f;
    uint32_t kw[UP][TT::QW], vw[TT::CH][TT::VW];
    int x = x0;
    int cur_id = x < count ? list[x] : 0;
    {
      size_t off = (((size_t)kv * n + cur_id) * B) * d;
      t.load(K + off, V + off, 0, kw, vw);
    }
    for (int t0 = 0; x < count;) {
      int nt0 = t0 + TT::CH;
      int nx = x;
      if (nt0 >= B) {
        nt0 = 0;
        nx = x + stride;
      }
      const bool have_next = nx < count;
      const int nid = have_next ? list[nx] : cur_id;
      const int lt0 = have_next ? nt0 : t0;
      size_t noff = (((size_t)kv * n + nid) * B) * d;
      uint32_t kn[UP][TT::QW], vn[TT::CH][TT::VW];
      t.load(K + noff, V + noff, lt0, kn, vn);
      t.template update<false, false>(qw, kw, vw, t0, B, scale, m, l, acc);
#pragma unroll
      for (int u = 0; u < UP; ++u)
#pragma unroll
        for (int c = 0; c < TT::QW; ++c) kw[u][c] = kn[u][c];
#pragma unroll
      for (int i = 0; i < TT::CH; ++i)
#pragma unroll
        for (int c = 0; c < TT::VW; ++c) vw[i][c] = vn[i][c];
      x = nx;
      t0 = nt0;
      cur_id = nid;
    }
    t.store(out, acc);
  }
};

// The repair of head h by one 512-thread workgroup.  lds_i: dynamic LDS laid
// out as map[N] (or pids[SP]) | ids[SA] | rows[SA] | wv[waves][D].
template <class Stream, int CHUNKS, bool VROW>
__device__ __forceinline__ void gqa_repair_head(const GqaRepairArgs& a, int h, int* lds_i,
                                                int* tmp, float* wm, float* wl, bool staged) {
  const int d = a.kv.d, n = a.kv.n;
  const bool use_map = n <= kRepairMapN;
  int* map = lds_i;
  int* pids = lds_i;
  int* ids = lds_i + (use_map ? n : a.sp);
  int* rows = ids + a.sa;
  float* wv = reinterpret_cast<float*>(rows + a.sa);
  int total_hit, nm;
  repair_membership(a, h, map, ids, rows, pids, tmp, &total_hit, &nm, staged);
  const int nrows = a.uni ? a.sp : total_hit;
  // ---- 2. roles
  const int nb = nm == 0 ? 0 : (nrows == 0 ? kRepairWaves : min(nm, kRepairWaves - 2));
  const int na = kRepairWaves - nb;
  const int w = wave_id();
  float m = -INFINITY, l = 0.f;
  if (w < na) {
    // A-wave: 4 row groups of 16 lanes; lane columns 8*lc + 128*c (+0..7)
    const float* pm = a.pm + (size_t)h * a.sp;
    const float* pl = a.pl + (size_t)h * a.sp;
    const int lc = lane_id() % kRowLanes;
    const int grp = w * (STK_WAVE / kRowLanes) + lane_id() / kRowLanes;
    const int ngroups = na * (STK_WAVE / kRowLanes);
    // rows per row group whose loads are in flight together
    constexpr int kRowBatch = CHUNKS >= 4 ? 2 : (CHUNKS == 2 ? 4 : 8);
    float acc[CHUNKS][8];
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[c][i] = 0.f;
    for (int r0 = grp; r0 < nrows; r0 += ngroups * kRowBatch) {
      float mm[kRowBatch], ll[kRowBatch], uu[kRowBatch][CHUNKS][8];
#pragma unroll
      for (int i = 0; i < kRowBatch; ++i) {
        int r = r0 + i * ngroups;
        bool on = r < nrows;
        int row = on ? (a.uni ? r : rows[r]) : 0;
        mm[i] = ld_or(pm, (int64_t)row, on, -INFINITY);
        ll[i] = ld_or(pl, (int64_t)row, on, 0.f);
        const float* ur = a.pu + ((size_t)h * a.sp + row) * d;
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c) {
          int col = 128 * c + 8 * lc;
          bool cv = col + 7 < d;
          if (VROW) {
            const float* src = ur + (cv ? col : 0);
            float4 x0 = *reinterpret_cast<const float4*>(src);
            float4 x1 = *reinterpret_cast<const float4*>(src + 4);
            uu[i][c][0] = x0.x; uu[i][c][1] = x0.y; uu[i][c][2] = x0.z; uu[i][c][3] = x0.w;
            uu[i][c][4] = x1.x; uu[i][c][5] = x1.y; uu[i][c][6] = x1.z; uu[i][c][7] = x1.w;
#pragma unroll
            for (int e = 0; e < 8; ++e) uu[i][c][e] = (on && cv) ? uu[i][c][e] : 0.f;
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) uu[i][c][e] = ld_or(ur, (int64_t)(col + e), on && col + e < d, 0.f);
          }
        }
      }
      float bm = mm[0];
#pragma unroll
      for (int i = 1; i < kRowBatch; ++i) bm = fmaxf(bm, mm[i]);
      float nmx = fmaxf(m, bm);
      if (nmx > m) {
        float alpha = wexp(m, nmx);
        l *= alpha;
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[c][e] *= alpha;
        m = nmx;
      }
#pragma unroll
      for (int i = 0; i < kRowBatch; ++i) {
        float wgt = wexp(mm[i], m);
        l += wgt * ll[i];
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[c][e] += wgt * uu[i][c][e];
      }
    }
    // merge the wave's 4 row groups (xor 16, 32)
#pragma unroll
    for (int off = kRowLanes; off < STK_WAVE; off <<= 1) {
      float om = __shfl_xor(m, off);
      float ol = __shfl_xor(l, off);
      float nmx = fmaxf(m, om);
      float f0 = wexp(m, nmx), f1 = wexp(om, nmx);
      l = l * f0 + ol * f1;
#pragma unroll
      for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[c][e] = acc[c][e] * f0 + __shfl_xor(acc[c][e], off) * f1;
      m = nmx;
    }
    if (lane_id() < kRowLanes) {
#pragma unroll
      for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          int col = 128 * c + 8 * lc + e;
          if (col < d) wv[w * d + col] = acc[c][e];
        }
    }
  } else {
    // B-wave: misses w - na, w - na + nb, ... with the online softmax
    Stream::run(a.kv, h, ids, w - na, nm, nb, m, l, wv + w * d);
  }
  if (lane_id() == 0) {
    wm[w] = m;
    wl[w] = l;
  }
  __syncthreads();
  // ---- 3. LSE merge of the wave states
  float M = -INFINITY;
#pragma unroll
  for (int x = 0; x < kRepairWaves; ++x) M = fmaxf(M, wm[x]);
  float f[kRepairWaves];
  float z = 0.f;
#pragma unroll
  for (int x = 0; x < kRepairWaves; ++x) {
    f[x] = wexp(wm[x], M);
    z += f[x] * wl[x];
  }
  for (int dd = threadIdx.x; dd < d; dd += blockDim.x) {
    float u = 0.f;
#pragma unroll
    for (int x = 0; x < kRepairWaves; ++x) u += f[x] * wv[x * d + dd];
    a.out[(size_t)h * d + dd] = u / z;
  }
}

inline size_t gqa_repair_lds(int n, int sa, int sp, int d) {
  size_t ints = (size_t)(n <= kRepairMapN ? n : sp) + 2 * (size_t)sa;
  return ints * 4 + (size_t)kRepairWaves * d * 4;
}

}  // namespace stk
