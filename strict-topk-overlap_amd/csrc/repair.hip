// Strict repair kernels: split (membership / saved merge / hybrid merge /
// wrong aggregate / fallback), fused single-launch repair, native-GQA
// saved/union merge and the single-launch light repair.
//
// Reference (6Mikao9/strict-topk-overlap):
//   strict_topk/kernels.py:120-247,359-407,504-550  split repair
//   strict_topk/fused.py:10-220                     repair_fused
//   strict_topk/gqa.py:62-104,384-413               repair_saved / repair_union
//   strict_topk/gqa_light.py:10-92                  repair_saved_light / auto
// Every kernel here runs one workgroup (4 waves) per query head.  KV blocks
// are read through the wave Tile routine; per-block states through weighted
// LDS reductions.  Query head h reads KV head h / (Hq / Hkv).
#include "gqa_repair.hpp"
#include "repair_fast.hpp"
#include "api.hpp"

namespace stk {

enum Mode : int { MODE_SAVED = 0, MODE_HYBRID = 1, MODE_COMPACT = 2 };

// ------------------------------------------------------------------ split
struct MembershipArgs {
  const void* p; int ptype; int sp;
  const void* a; int atype; int sa;
  const uint8_t* high;          // [h, sp] (hybrid, compact)
  const void* rids; int sc;     // compact retained IDs [h, sc] (ptype)
  int mode;
  uint8_t* hit; uint8_t* miss; uint8_t* wrong; uint8_t* low_hit;
};

__global__ __launch_bounds__(256) void k_membership(MembershipArgs a) {
  __shared__ HeadLds s;
  int h = blockIdx.x;
  stage_ids(a.p, a.ptype, (int64_t)h * a.sp, a.sp, s.p);
  stage_ids(a.a, a.atype, (int64_t)h * a.sa, a.sa, s.a);
  __syncthreads();
  membership(s, a.sp, a.sa);
  for (int i = threadIdx.x; i < a.sa; i += blockDim.x) a.miss[(size_t)h * a.sa + i] = s.fa[i];
  int lowhit = 0;
  if (a.mode != MODE_SAVED)
    for (int i = threadIdx.x; i < a.sp; i += blockDim.x)
      lowhit |= s.fp[i] && !a.high[(size_t)h * a.sp + i];
  lowhit = block_or(lowhit, s.ired);
  for (int i = threadIdx.x; i < a.sp; i += blockDim.x) {
    bool phit = s.fp[i];
    bool high = a.mode != MODE_SAVED && a.high[(size_t)h * a.sp + i];
    a.wrong[(size_t)h * a.sp + i] = a.mode != MODE_SAVED && !phit && !high && lowhit;
    if (a.mode == MODE_SAVED) a.hit[(size_t)h * a.sp + i] = phit;
    else if (a.mode == MODE_HYBRID) a.hit[(size_t)h * a.sp + i] = phit && high;
  }
  if (a.mode == MODE_COMPACT) {
    for (int c = threadIdx.x; c < a.sc; c += blockDim.x) {
      int64_t r = load_id(a.rids, a.ptype, (int64_t)h * a.sc + c);
      bool f = false;
      if (r >= 0)
        for (int j = 0; j < a.sa; ++j) f |= (s.a[j] == r);
      a.hit[(size_t)h * a.sc + c] = f;
    }
  }
  if (threadIdx.x == 0) a.low_hit[h] = lowhit;
}

struct MergeRepairArgs {
  int h, sp, sa, sc, sw, d;
  const float* pm; const float* pl; const float* pu; const uint8_t* hit;   // [h, sc]
  const float* am; const float* al; const float* au;                      // [h, sa]
  const float* lm; const float* ll; const float* lu; const float* labs;   // low
  const uint8_t* low_hit;
  const float* wm; const float* wl; const float* wu;                      // [h, sw]
  float min_remain, cancel;
  float* out; uint8_t* bad; float* remain;
};

// strict_topk/kernels.py:146-168
__global__ __launch_bounds__(256) void k_saved_merge(MergeRepairArgs a) {
  __shared__ HeadLds s;
  int h = blockIdx.x;
  const float* pm = a.pm + (size_t)h * a.sc;
  const float* am = a.am + (size_t)h * a.sa;
  const uint8_t* hit = a.hit + (size_t)h * a.sc;
  float mx = -INFINITY;
  for (int j = threadIdx.x; j < a.sc; j += blockDim.x) if (hit[j]) mx = fmaxf(mx, pm[j]);
  for (int j = threadIdx.x; j < a.sa; j += blockDim.x) mx = fmaxf(mx, am[j]);
  mx = block_max(mx, s.red);
  float z1 = sum_states(
      s, a.sc, a.d, [&](int j) { return hit[j] ? wexp(pm[j], mx) : 0.f; },
      [&](int j) { return a.pl[(size_t)h * a.sc + j]; },
      [&](int j) { return a.pu + ((size_t)h * a.sc + j) * a.d; }, s.u0);
  float z2 = sum_states(
      s, a.sa, a.d, [&](int j) { return wexp(am[j], mx); },
      [&](int j) { return a.al[(size_t)h * a.sa + j]; },
      [&](int j) { return a.au + ((size_t)h * a.sa + j) * a.d; }, s.u1);
  float z = z1 + z2;
  for (int dd = threadIdx.x; dd < a.d; dd += blockDim.x)
    a.out[(size_t)h * a.d + dd] = (s.u0[dd] + s.u1[dd]) / z;
  if (threadIdx.x == 0) {
    a.bad[h] = 0;
    a.remain[h] = 1.f;
  }
}

// strict_topk/kernels.py:171-220
__global__ __launch_bounds__(256) void k_hybrid_merge(MergeRepairArgs a) {
  __shared__ HeadLds s;
  int h = blockIdx.x;
  const float* pm = a.pm + (size_t)h * a.sc;
  const float* am = a.am + (size_t)h * a.sa;
  const float* wm = a.wm + (size_t)h * a.sw;
  const uint8_t* hit = a.hit + (size_t)h * a.sc;
  bool low_hit = a.low_hit[h] != 0;
  float lm = a.lm[h];
  float mx = -INFINITY;
  for (int j = threadIdx.x; j < a.sc; j += blockDim.x) if (hit[j]) mx = fmaxf(mx, pm[j]);
  for (int j = threadIdx.x; j < a.sa; j += blockDim.x) mx = fmaxf(mx, am[j]);
  mx = block_max(mx, s.red);
  if (low_hit) mx = fmaxf(mx, lm);
  float zp = sum_states(
      s, a.sc, a.d, [&](int j) { return hit[j] ? wexp(pm[j], mx) : 0.f; },
      [&](int j) { return a.pl[(size_t)h * a.sc + j]; },
      [&](int j) { return a.pu + ((size_t)h * a.sc + j) * a.d; }, s.u0);
  float za = sum_states(
      s, a.sa, a.d, [&](int j) { return wexp(am[j], mx); },
      [&](int j) { return a.al[(size_t)h * a.sa + j]; },
      [&](int j) { return a.au + ((size_t)h * a.sa + j) * a.d; }, s.u1);
  float removed = 0.f;
  if (low_hit)
    removed = sum_states(
        s, a.sw, a.d, [&](int j) { return wexp(wm[j], mx); },
        [&](int j) { return a.wl[(size_t)h * a.sw + j]; },
        [&](int j) { return a.wu + ((size_t)h * a.sw + j) * a.d; }, s.u2);
  else
    for (int dd = threadIdx.x; dd < a.d; dd += blockDim.x) s.u2[dd] = 0.f;
  __syncthreads();
  float lowalpha = low_hit ? expf(lm - mx) : 0.f;
  float ll = (low_hit ? a.ll[h] : 0.f) * lowalpha;
  float remaining = ll - removed;
  float fraction = ll > 0.f ? remaining / fmaxf(ll, 1e-30f) : 1.f;
  float z = remaining + zp + za;
  int cancel = 0, nonfinite = 0;
  for (int dd = threadIdx.x; dd < a.d; dd += blockDim.x) {
    float lu = (low_hit ? a.lu[(size_t)h * a.d + dd] : 0.f) * lowalpha;
    float ru = s.u2[dd];
    float residual = lu - ru;
    float lab = (low_hit ? a.labs[(size_t)h * a.d + dd] : 0.f) * lowalpha;
    float sc = lab + fabsf(ru);
    cancel |= (fabsf(residual) < a.cancel * sc) && (sc > 0.f) && low_hit;
    float o = (residual + s.u0[dd] + s.u1[dd]) / fmaxf(z, 1e-30f);
    nonfinite |= is_bad(o);
    a.out[(size_t)h * a.d + dd] = o;
  }
  cancel = block_or(cancel, s.ired);
  nonfinite = block_or(nonfinite, s.ired);
  bool bad = (z <= 0.f) || (fraction < a.min_remain) || (fraction != fraction) ||
             (fabsf(z) == INFINITY) || cancel || nonfinite;
  if (threadIdx.x == 0) {
    a.bad[h] = bad;
    a.remain[h] = fraction;
  }
}

struct StreamArgs {
  KV kv;
  const void* ids; int itype; int s;
  const uint8_t* flags;      // per-id activity (wrong aggregate) or per-head (fallback)
  const float* lm;           // fixed frame (wrong aggregate)
  float* m; float* l; float* u;   // outputs
  float* out;
};

// strict_topk/kernels.py:384-407: wrong blocks of P aggregated in the low frame
template <typename T, int VEC, int NC, int U>
__global__ __launch_bounds__(256) void k_wrong_aggregate(StreamArgs a) {
  using TL = Tile<T, VEC, NC>;
  __shared__ HeadLds s;
  int h = blockIdx.x;
  int kv = h / (a.kv.hq / a.kv.hkv);
  TL t;
  t.init(a.kv.d);
  float qr[TL::R];
  t.load_q(reinterpret_cast<const T*>(a.kv.q) + (size_t)h * a.kv.d, qr);
  float lm = a.lm[h];
  float m, z;
  stream_blocks<T, VEC, NC, U, true>(
      s, qr, t, (const T*)a.kv.k, (const T*)a.kv.v, kv, a.kv.n, a.kv.b, a.kv.d, a.s,
      [&](int j) -> int64_t {
        return a.flags[(size_t)h * a.s + j] ? load_id(a.ids, a.itype, (int64_t)h * a.s + j) : -1;
      },
      lm, m, z, s.u0);
  for (int dd = threadIdx.x; dd < a.kv.d; dd += blockDim.x) a.u[(size_t)h * a.kv.d + dd] = s.u0[dd];
  if (threadIdx.x == 0) {
    a.m[h] = lm;
    a.l[h] = z;
  }
}

// strict_topk/kernels.py:223-247: strict online softmax over A on bad heads
template <typename T, int VEC, int NC, int U>
__global__ __launch_bounds__(256) void k_fallback(StreamArgs a) {
  using TL = Tile<T, VEC, NC>;
  __shared__ HeadLds s;
  int h = blockIdx.x;
  if (!a.flags[h]) return;
  int kv = h / (a.kv.hq / a.kv.hkv);
  TL t;
  t.init(a.kv.d);
  float qr[TL::R];
  t.load_q(reinterpret_cast<const T*>(a.kv.q) + (size_t)h * a.kv.d, qr);
  float m, z;
  stream_blocks<T, VEC, NC, U, false>(
      s, qr, t, (const T*)a.kv.k, (const T*)a.kv.v, kv, a.kv.n, a.kv.b, a.kv.d, a.s,
      [&](int j) -> int64_t { return load_id(a.ids, a.itype, (int64_t)h * a.s + j); }, 0.f, m,
      z, s.u0);
  for (int dd = threadIdx.x; dd < a.kv.d; dd += blockDim.x)
    a.out[(size_t)h * a.kv.d + dd] = s.u0[dd] / z;
}

// ------------------------------------------------------------------ fused
struct FusedArgs {
  KV kv;
  const void* a; int atype; int sa;
  const void* p; int ptype; int sp;
  int sc, mode;
  const float* pm; const float* pl; const float* pu;
  const uint8_t* high; const void* rids;
  const float* lm; const float* ll; const float* lu; const float* labs;
  const float* mass_m; const float* mass_l;
  float min_remain, cancel, eps;
  float* out; uint8_t* bad; float* remain; uint8_t* approx; float* extra;
};

// strict_topk/fused.py:48-173
template <typename T, int VEC, int NC, int U>
__global__ __launch_bounds__(256) void k_repair_fused(FusedArgs a) {
  using TL = Tile<T, VEC, NC>;
  __shared__ HeadLds s;
  __shared__ uint8_t keep[kMaxIds];
  const int h = blockIdx.x;
  const int d = a.kv.d;
  const int kv = h / (a.kv.hq / a.kv.hkv);
  const bool hybrid = a.mode != MODE_SAVED;
  const bool compact = a.mode == MODE_COMPACT;
  stage_ids(a.p, a.ptype, (int64_t)h * a.sp, a.sp, s.p);
  stage_ids(a.a, a.atype, (int64_t)h * a.sa, a.sa, s.a);
  __syncthreads();
  membership(s, a.sp, a.sa);   // fp = hit over P, fa = missing over A
  const uint8_t* high = hybrid ? a.high + (size_t)h * a.sp : nullptr;
  int lowhit = 0;
  if (hybrid)
    for (int i = threadIdx.x; i < a.sp; i += blockDim.x) lowhit |= s.fp[i] && !high[i];
  lowhit = block_or(lowhit, s.ired);
  if (compact) {
    for (int c = threadIdx.x; c < a.sc; c += blockDim.x) {
      int64_t r = load_id(a.rids, a.ptype, (int64_t)h * a.sc + c);
      bool f = false;
      for (int j = 0; j < a.sa; ++j) f |= (s.a[j] == r);
      keep[c] = f;
    }
  } else {
    for (int c = threadIdx.x; c < a.sp; c += blockDim.x)
      keep[c] = s.fp[c] && (!hybrid || high[c]);
  }
  __syncthreads();
  const float* pm = a.pm + (size_t)h * a.sc;
  const float* pl = a.pl + (size_t)h * a.sc;
  float rmax = -INFINITY;
  for (int c = threadIdx.x; c < a.sc; c += blockDim.x) if (keep[c]) rmax = fmaxf(rmax, pm[c]);
  rmax = block_max(rmax, s.red);

  TL t;
  t.init(d);
  float qr[TL::R];
  t.load_q(reinterpret_cast<const T*>(a.kv.q) + (size_t)h * d, qr);
  const T* K = (const T*)a.kv.k;
  const T* V = (const T*)a.kv.v;

  float fraction = 1.f, mass = 0.f, lm = -INFINITY, extra_bound = 0.f;
  bool bad = false, skip = false;
  for (int dd = threadIdx.x; dd < d; dd += blockDim.x) s.u1[dd] = 0.f;   // residual
  __syncthreads();
  if (hybrid && lowhit) {
    lm = a.lm[h];
    float ll = a.ll[h];
    // wrong = ~hit & ~high over P positions
    int wcount = 0;
    for (int i = threadIdx.x; i < a.sp; i += blockDim.x) wcount += !s.fp[i] && !high[i];
    wcount = (int)block_sum((float)wcount, s.red);
    if (a.eps > 0.f && wcount > 0) {
      float ref = fmaxf(rmax, lm);
      float wmass = 0.f, den = 0.f;
      for (int i = threadIdx.x; i < a.sp; i += blockDim.x)
        if (!s.fp[i] && !high[i]) wmass += wexp(a.mass_m[(size_t)h * a.sp + i], ref) * a.mass_l[(size_t)h * a.sp + i];
      for (int c = threadIdx.x; c < a.sc; c += blockDim.x)
        if (keep[c]) den += wexp(pm[c], ref) * pl[c];
      wmass = block_sum(wmass, s.red);
      den = block_sum(den, s.red);
      den += expf(lm - ref) * ll;
      extra_bound = wmass / den;
      skip = extra_bound <= a.eps;
    }
    float removed = 0.f;
    for (int dd = threadIdx.x; dd < d; dd += blockDim.x) s.u2[dd] = 0.f;
    __syncthreads();
    if (wcount > 0 && !skip) {
      float mm;
      stream_blocks<T, VEC, NC, U, true>(
          s, qr, t, K, V, kv, a.kv.n, a.kv.b, d, a.sp,
          [&](int j) -> int64_t { return (!s.fp[j] && !high[j]) ? s.p[j] : -1; }, lm, mm,
          removed, s.u2);
    }
    mass = ll - removed;
    fraction = mass / ll;
    int cancel = 0;
    for (int dd = threadIdx.x; dd < d; dd += blockDim.x) {
      float ru = s.u2[dd];
      float residual = a.lu[(size_t)h * d + dd] - ru;
      s.u1[dd] = residual;
      float sc = a.labs[(size_t)h * d + dd] + fabsf(ru);
      cancel |= (fabsf(residual) < a.cancel * sc) && (sc > 0.f);
    }
    cancel = block_or(cancel, s.ired);
    bad = (fraction < a.min_remain) || (fraction != fraction) || cancel;
  }
  float mx = fmaxf(rmax, lm);
  float ref = mx == -INFINITY ? 0.f : mx;
  float zr = sum_states(
      s, a.sc, d, [&](int c) { return keep[c] ? wexp(pm[c], ref) : 0.f; },
      [&](int c) { return pl[c]; }, [&](int c) { return a.pu + ((size_t)h * a.sc + c) * d; },
      s.u0);
  float low_alpha = lm == -INFINITY ? 0.f : expf(lm - ref);
  float z = zr + low_alpha * mass;
  for (int dd = threadIdx.x; dd < d; dd += blockDim.x) s.u0[dd] += low_alpha * s.u1[dd];
  __syncthreads();
  bool all = hybrid && bad;
  if (all) {
    mx = -INFINITY;
    z = 0.f;
    for (int dd = threadIdx.x; dd < d; dd += blockDim.x) s.u0[dd] = 0.f;
    __syncthreads();
  }
  int todo = 0;
  for (int i = threadIdx.x; i < a.sa; i += blockDim.x) todo += all || s.fa[i];
  todo = (int)block_sum((float)todo, s.red);
  if (todo > 0) {
    float mw, zw;
    stream_blocks<T, VEC, NC, U, false>(
        s, qr, t, K, V, kv, a.kv.n, a.kv.b, d, a.sa,
        [&](int j) -> int64_t { return (all || s.fa[j]) ? s.a[j] : -1; }, 0.f, mw, zw, s.u1);
    float M = fmaxf(mx, mw);
    float f0 = wexp(mx, M), f1 = wexp(mw, M);
    z = z * f0 + zw * f1;
    for (int dd = threadIdx.x; dd < d; dd += blockDim.x) s.u0[dd] = s.u0[dd] * f0 + s.u1[dd] * f1;
    __syncthreads();
  }
  int invalid = 0;
  for (int dd = threadIdx.x; dd < d; dd += blockDim.x) invalid |= is_bad(s.u0[dd] / z);
  invalid = block_or(invalid, s.ired);
  bool redo = false;
  if (hybrid) {
    bool bad_out = (z <= 0.f) || (fabsf(z) == INFINITY) || invalid;
    redo = bad_out && !bad;
    bad = bad || bad_out;
  }
  if (redo) {
    float mw, zw;
    stream_blocks<T, VEC, NC, U, false>(
        s, qr, t, K, V, kv, a.kv.n, a.kv.b, d, a.sa, [&](int j) -> int64_t { return s.a[j]; },
        0.f, mw, zw, s.u0);
    z = zw;
  }
  for (int dd = threadIdx.x; dd < d; dd += blockDim.x) a.out[(size_t)h * d + dd] = s.u0[dd] / z;
  if (threadIdx.x == 0) {
    a.bad[h] = bad;
    a.remain[h] = fraction;
    if (a.eps > 0.f) {
      bool used = skip && !bad;
      a.approx[h] = used;
      a.extra[h] = used ? extra_bound : 0.f;
    }
  }
}


template <class Stream, int CHUNKS, bool VROW>
__global__ __launch_bounds__(kRepairThreads) void k_gqa_repair(GqaRepairArgs a) {
  extern __shared__ int lds_i[];
  __shared__ int tmp[kRepairWaves];
  __shared__ float wm[kRepairWaves], wl[kRepairWaves];
  gqa_repair_head<Stream, CHUNKS, VROW>(a, xcd_remap(blockIdx.x, gridDim.x), lds_i, tmp, wm, wl, false);
}

}  // namespace stk

using namespace stk;

static StkCheck check_ids(int sa, int sp) {
  if (sa <= 0 || sp <= 0) return {false, "ids must be nonempty"};
  if (sa > kMaxIds || sp > kMaxIds) return {false, "at most 4096 IDs per row are supported"};
  return {true, ""};
}

extern "C" {

// Strict recompute of the selected set on flagged heads (kernels.py:223-247).
STK_API int stk_fallback(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                         int n, int b, int d, const void* selected, int sel_dtype, int sa,
                         const uint8_t* flags, float* out, void* stream) {
  STK_REQUIRE(stk_check_kv(dtype, hq, hkv, n, b, d));
  STK_REQUIRE(q && k && v && selected && flags && out, "null pointer");
  KV kvd{q, k, v, hq, hkv, n, b, d};
  StreamArgs fb{kvd, selected, sel_dtype, sa, flags, nullptr, nullptr, nullptr, nullptr, out};
  hipStream_t st = (hipStream_t)stream;
  STK_DISPATCH_TILE(dtype, d, {
    hipLaunchKernelGGL((k_fallback<T, VEC, NC, U>), dim3(hq), dim3(256), 0, st, fb);
  });
  return stk_check_launch("k_fallback");
}

STK_API size_t stk_repair_workspace_bytes(int hq, int sa, int sp, int sc, int d, int mode) {
  size_t b = 0;
  b += stk_align((size_t)hq * sc);            // hit
  b += stk_align((size_t)hq * sa);            // miss
  b += stk_align((size_t)hq * sp);            // wrong
  b += stk_align((size_t)hq);                 // low_hit
  b += stk_align((size_t)hq * sa * 4) * 2 + stk_align((size_t)hq * sa * d * 4);   // miss states
  int sw = mode == MODE_COMPACT ? 1 : sp;
  if (mode != MODE_SAVED)
    b += stk_align((size_t)hq * sw * 4) * 2 + stk_align((size_t)hq * sw * d * 4);
  return b;
}

// strict_topk/kernels.py:504-550
STK_API int stk_repair(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                       int n, int b, int d, const void* selected, int sel_dtype, int sa,
                       const void* predicted, int pred_dtype, int sp, int mode, int sc,
                       const float* pm, const float* pl, const float* pu, const uint8_t* high,
                       const float* low_m, const float* low_l, const float* low_u,
                       const float* low_abs, const void* retained_ids, float min_remaining,
                       float cancellation_tol, float* out, uint8_t* fallback, float* remaining,
                       void* workspace, size_t workspace_bytes, void* stream) {
  STK_REQUIRE(stk_check_kv(dtype, hq, hkv, n, b, d));
  STK_REQUIRE(check_ids(sa, sp));
  STK_REQUIRE(mode >= 0 && mode <= 2, "bad prediction mode");
  STK_REQUIRE(q && k && v && selected && predicted && pm && pl && pu && out && fallback &&
                  remaining,
              "null pointer");
  STK_REQUIRE(mode == MODE_SAVED || (high && low_m && low_l && low_u && low_abs), "null low group");
  STK_REQUIRE(mode != MODE_COMPACT || retained_ids, "null retained ids");
  STK_REQUIRE(sc > 0 && sc <= kMaxIds, "bad prediction state width");
  STK_REQUIRE(workspace && workspace_bytes >= stk_repair_workspace_bytes(hq, sa, sp, sc, d, mode),
              "workspace too small");
  hipStream_t st = (hipStream_t)stream;
  Carve w(workspace);
  uint8_t* hit = w.take<uint8_t>((size_t)hq * sc);
  uint8_t* miss = w.take<uint8_t>((size_t)hq * sa);
  uint8_t* wrong = w.take<uint8_t>((size_t)hq * sp);
  uint8_t* low_hit = w.take<uint8_t>((size_t)hq);
  float* am = w.take<float>((size_t)hq * sa);
  float* al = w.take<float>((size_t)hq * sa);
  float* au = w.take<float>((size_t)hq * sa * d);
  MembershipArgs ma{predicted, pred_dtype, sp, selected, sel_dtype, sa, high, retained_ids, sc,
                    mode, hit, miss, wrong, low_hit};
  hipLaunchKernelGGL(k_membership, dim3(hq), dim3(256), 0, st, ma);
  int rc = stk_check_launch("k_membership");
  if (rc) return rc;
  rc = stk_launch_states(q, k, v, dtype, hq, hkv, n, b, d, selected, sel_dtype, sa, miss, 2,
                         nullptr, 0, 0, nullptr, am, al, au, true, st);
  if (rc) return rc;
  MergeRepairArgs mr{};
  mr.h = hq; mr.sp = sp; mr.sa = sa; mr.sc = sc; mr.d = d;
  mr.pm = pm; mr.pl = pl; mr.pu = pu; mr.hit = hit;
  mr.am = am; mr.al = al; mr.au = au;
  mr.out = out; mr.bad = fallback; mr.remain = remaining;
  if (mode == MODE_SAVED) {
    hipLaunchKernelGGL(k_saved_merge, dim3(hq), dim3(256), 0, st, mr);
    return stk_check_launch("k_saved_merge");
  }
  int sw = mode == MODE_COMPACT ? 1 : sp;
  float* wm = w.take<float>((size_t)hq * sw);
  float* wl = w.take<float>((size_t)hq * sw);
  float* wu = w.take<float>((size_t)hq * sw * d);
  KV kvd{q, k, v, hq, hkv, n, b, d};
  if (mode == MODE_COMPACT) {
    StreamArgs sa_{kvd, predicted, pred_dtype, sp, wrong, low_m, wm, wl, wu, nullptr};
    STK_DISPATCH_TILE(dtype, d, {
      hipLaunchKernelGGL((k_wrong_aggregate<T, VEC, NC, U>), dim3(hq), dim3(256), 0, st, sa_);
    });
    rc = stk_check_launch("k_wrong_aggregate");
  } else {
    rc = stk_launch_states(q, k, v, dtype, hq, hkv, n, b, d, predicted, pred_dtype, sp, wrong, 2,
                           nullptr, 0, 0, nullptr, wm, wl, wu, true, st);
  }
  if (rc) return rc;
  mr.sw = sw; mr.wm = wm; mr.wl = wl; mr.wu = wu;
  mr.lm = low_m; mr.ll = low_l; mr.lu = low_u; mr.labs = low_abs; mr.low_hit = low_hit;
  mr.min_remain = min_remaining; mr.cancel = cancellation_tol;
  hipLaunchKernelGGL(k_hybrid_merge, dim3(hq), dim3(256), 0, st, mr);
  rc = stk_check_launch("k_hybrid_merge");
  if (rc) return rc;
  return stk_fallback(q, k, v, dtype, hq, hkv, n, b, d, selected, sel_dtype, sa, fallback, out,
                      stream);
}

// strict_topk/fused.py:176-220
STK_API int stk_repair_fused(const void* q, const void* k, const void* v, int dtype, int hq,
                             int hkv, int n, int b, int d, const void* selected, int sel_dtype,
                             int sa, const void* predicted, int pred_dtype, int sp, int mode,
                             int sc, const float* pm, const float* pl, const float* pu,
                             const uint8_t* high, const float* low_m, const float* low_l,
                             const float* low_u, const float* low_abs, const void* retained_ids,
                             const float* mass_m, const float* mass_l, float min_remaining,
                             float cancellation_tol, float max_extra_mass, float* out,
                             uint8_t* fallback, float* remaining, uint8_t* approximate,
                             float* extra_mass_bound, void* stream) {
  STK_REQUIRE(stk_check_kv(dtype, hq, hkv, n, b, d));
  STK_REQUIRE(check_ids(sa, sp));
  STK_REQUIRE(mode >= 0 && mode <= 2, "bad prediction mode");
  STK_REQUIRE(q && k && v && selected && predicted && pm && pl && pu && out && fallback &&
                  remaining,
              "null pointer");
  STK_REQUIRE(mode == MODE_SAVED || (high && low_m && low_l && low_u && low_abs), "null low group");
  STK_REQUIRE(mode != MODE_COMPACT || retained_ids, "null retained ids");
  STK_REQUIRE(sc > 0 && sc <= kMaxIds, "bad prediction state width");
  STK_REQUIRE(max_extra_mass >= 0.f && max_extra_mass <= 1.f, "max_extra_mass must be in [0, 1]");
  STK_REQUIRE(max_extra_mass == 0.f || (approximate && extra_mass_bound), "null budget outputs");
  STK_REQUIRE(max_extra_mass == 0.f || mode == MODE_SAVED || (mass_m && mass_l),
              "positive max_extra_mass requires speculate(..., keep_mass=True)");
  FusedArgs f{};
  f.kv = KV{q, k, v, hq, hkv, n, b, d};
  f.a = selected; f.atype = sel_dtype; f.sa = sa;
  f.p = predicted; f.ptype = pred_dtype; f.sp = sp; f.sc = sc; f.mode = mode;
  f.pm = pm; f.pl = pl; f.pu = pu; f.high = high; f.rids = retained_ids;
  f.lm = low_m; f.ll = low_l; f.lu = low_u; f.labs = low_abs; f.mass_m = mass_m; f.mass_l = mass_l;
  f.min_remain = min_remaining; f.cancel = cancellation_tol; f.eps = max_extra_mass;
  f.out = out; f.bad = fallback; f.remain = remaining; f.approx = approximate;
  f.extra = extra_mass_bound;
  hipStream_t st = (hipStream_t)stream;
  STK_DISPATCH_TILE(dtype, d, {
    hipLaunchKernelGGL((k_repair_fused<T, VEC, NC, U>), dim3(hq), dim3(256), 0, st, f);
  });
  return stk_check_launch("k_repair_fused");
}

STK_API size_t stk_gqa_repair_workspace_bytes(int hq, int sa, int d) {
  (void)hq; (void)sa; (void)d;
  return 0;   // the single-launch repair keeps its scratch in LDS
}

static int launch_gqa_repair(const GqaRepairArgs& g, int dtype, hipStream_t st) {
  // the one-workgroup repair (repair_fast.hpp) where it covers the shape
  const int rc = launch_repair_fast(g, dtype, st);
  if (rc <= 0) return rc;
  const int d = g.kv.d;
  size_t lds = gqa_repair_lds(g.kv.n, g.sa, g.sp, d);
  if (lds > 160 * 1024) {
    stk_set_error("repair scratch of %zu bytes exceeds the 160 KiB LDS", lds);
    return STK_EINVAL;
  }
  const bool vrow = d % 8 == 0 && (reinterpret_cast<uintptr_t>(g.pu) & 15) == 0;
  const uintptr_t align = reinterpret_cast<uintptr_t>(g.kv.q) | reinterpret_cast<uintptr_t>(g.kv.k) |
                          reinterpret_cast<uintptr_t>(g.kv.v);
  const int nch = tok_nch(dtype, d, g.kv.b, align);
  const dim3 grid(g.kv.hq), block(kRepairThreads);
  if (nch) {
    // d is 64, 128 or 256 here
    const bool one = tok_up(g.kv.b) == 1;
#define STK_REPAIR_TOK(UPV)                                                                           \
    STK_DISPATCH_TOK(dtype, nch, {                                                                    \
      if (d <= 128 && vrow)                                                                           \
        hipLaunchKernelGGL((k_gqa_repair<TokStream<T, NCH, UPV>, 1, true>), grid, block, lds, st, g);  \
      else if (d <= 128)                                                                              \
        hipLaunchKernelGGL((k_gqa_repair<TokStream<T, NCH, UPV>, 1, false>), grid, block, lds, st, g); \
      else if (vrow)                                                                                  \
        hipLaunchKernelGGL((k_gqa_repair<TokStream<T, NCH, UPV>, 2, true>), grid, block, lds, st, g);  \
      else                                                                                            \
        hipLaunchKernelGGL((k_gqa_repair<TokStream<T, NCH, UPV>, 2, false>), grid, block, lds, st, g); \
    })
    if (one) STK_REPAIR_TOK(1);
    else STK_REPAIR_TOK(2);
#undef STK_REPAIR_TOK
    return stk_check_launch("k_gqa_repair");
  }
#define STK_REPAIR_CH(CH)                                                                                 \
  STK_DISPATCH_TILE(dtype, d, {                                                                           \
    if (vrow)                                                                                             \
      hipLaunchKernelGGL((k_gqa_repair<GenericStream<T, VEC, NC, U>, CH, true>), grid, block, lds, st, g); \
    else                                                                                                  \
      hipLaunchKernelGGL((k_gqa_repair<GenericStream<T, VEC, NC, U>, CH, false>), grid, block, lds, st, g); \
  })
  if (d <= 128) STK_REPAIR_CH(1);
  else if (d <= 256) STK_REPAIR_CH(2);
  else if (d <= 512) STK_REPAIR_CH(4);
  else STK_REPAIR_CH(8);
#undef STK_REPAIR_CH
  return stk_check_launch("k_gqa_repair");
}

// strict_topk/gqa.py:164-193 (saved / union), single launch
STK_API int stk_gqa_repair(const void* q, const void* k, const void* v, int dtype, int hq,
                           int hkv, int n, int b, int d, const void* selected, int sel_dtype,
                           int sa, const void* predicted, int pred_dtype, int sp, const float* pm,
                           const float* pl, const float* pu, int union_mode, float* out,
                           void* workspace, size_t workspace_bytes, void* stream) {
  (void)workspace; (void)workspace_bytes;
  STK_REQUIRE(stk_check_kv(dtype, hq, hkv, n, b, d));
  STK_REQUIRE(check_ids(sa, sp));
  STK_REQUIRE(q && k && v && selected && predicted && pm && pl && pu && out, "null pointer");
  GqaRepairArgs g{KV{q, k, v, hq, hkv, n, b, d}, selected, sel_dtype, sa, predicted, pred_dtype,
                  sp, pm, pl, pu, union_mode ? 1 : 0, out};
  return launch_gqa_repair(g, dtype, (hipStream_t)stream);
}

// strict_topk/gqa_light.py:63-77: the same single-launch strict repair
STK_API int stk_repair_light(const void* q, const void* k, const void* v, int dtype, int hq,
                             int hkv, int n, int b, int d, const void* selected, int sel_dtype,
                             int sa, const void* predicted, int pred_dtype, int sp,
                             const float* pm, const float* pl, const float* pu, float* out,
                             void* stream) {
  STK_REQUIRE(stk_check_kv(dtype, hq, hkv, n, b, d));
  STK_REQUIRE(check_ids(sa, sp));
  STK_REQUIRE(q && k && v && selected && predicted && pm && pl && pu && out, "null pointer");
  GqaRepairArgs g{KV{q, k, v, hq, hkv, n, b, d}, selected, sel_dtype, sa, predicted, pred_dtype,
                  sp, pm, pl, pu, 0, out};
  return launch_gqa_repair(g, dtype, (hipStream_t)stream);
}

}  // extern "C"
