// Signed add/erase repair: job-queue schedule, per-job signed block states,
// and the guarded merges.
//
// Reference (6Mikao9/strict-topk-overlap):
//   strict_topk/signed_repair.py:18-82    _schedule        -> k_schedule
//   strict_topk/signed_repair.py:85-109   _signed_partials -> k_jobs (SIGNED)
//   strict_topk/signed_repair.py:112-172  _merge           -> k_signed_merge
//   strict_topk/signed_fused.py:30-67     _corrections     -> k_jobs (FUSED)
//   strict_topk/signed_fused.py:70-145    _finalize        -> k_finalize
// Queue rows hold misses first (selected-position order) and then the
// wrong low blocks (predicted-position order); job counts are per head, and
// the per-job kernel exits early past a head's count, so a captured graph
// does not depend on the data.
#include "head.hpp"
#include "api.hpp"
#include "srepair.hpp"

namespace stk {

enum { MODE_SAVED = 0, MODE_HYBRID = 1, MODE_COMPACT = 2 };

struct SchedArgs {
  const void* a; int atype; int sa;
  const void* p; int ptype; int sp;
  int sc, mode, cap;
  const uint8_t* high; const void* rids;
  const float* pm; const float* pl;   // prediction state m, l [h, sc]
  const float* lm; const float* ll;
  const float* mass_m; const float* mass_l;
  float eps;
  void* queue; int qtype;
  int32_t* pos; int32_t* total; uint8_t* keep; uint8_t* low_hit;
  uint8_t* approx; float* extra;
};

__global__ __launch_bounds__(256) void k_schedule(SchedArgs a) {
  __shared__ HeadLds s;
  __shared__ int rk[kMaxIds];
  __shared__ int scan[kThreads];
  __shared__ uint8_t wrong[kMaxIds];
  const int h = blockIdx.x;
  const bool hybrid = a.mode != MODE_SAVED;
  const bool compact = a.mode == MODE_COMPACT;
  stage_ids(a.p, a.ptype, (int64_t)h * a.sp, a.sp, s.p);
  stage_ids(a.a, a.atype, (int64_t)h * a.sa, a.sa, s.a);
  __syncthreads();
  membership(s, a.sp, a.sa);
  int nmiss = rank_flags(s.fa, a.sa, rk, scan);
  for (int i = threadIdx.x; i < a.sa; i += blockDim.x)
    if (s.fa[i]) store_id(a.queue, a.qtype, (int64_t)h * a.cap + rk[i], s.a[i]);
  const uint8_t* high = hybrid ? a.high + (size_t)h * a.sp : nullptr;
  int lowhit = 0;
  if (hybrid)
    for (int i = threadIdx.x; i < a.sp; i += blockDim.x) lowhit |= s.fp[i] && !high[i];
  lowhit = block_or(lowhit, s.ired);
  for (int i = threadIdx.x; i < a.sp; i += blockDim.x)
    wrong[i] = hybrid && lowhit && !s.fp[i] && !high[i];
  if (compact) {
    for (int c = threadIdx.x; c < a.sc; c += blockDim.x) {
      int64_t r = load_id(a.rids, a.ptype, (int64_t)h * a.sc + c);
      bool f = false;
      for (int j = 0; j < a.sa; ++j) f |= (s.a[j] == r);
      a.keep[(size_t)h * a.sc + c] = f;
    }
  } else {
    for (int c = threadIdx.x; c < a.sp; c += blockDim.x)
      a.keep[(size_t)h * a.sc + c] = s.fp[c] && (!hybrid || high[c]);
  }
  __syncthreads();
  bool skip = false;
  float extra = 0.f;
  int total = nmiss;
  if (hybrid) {
    int nw = 0;
    for (int i = threadIdx.x; i < a.sp; i += blockDim.x) nw += wrong[i];
    nw = (int)block_sum((float)nw, s.red);
    if (a.eps > 0.f && nw > 0) {
      float lm = a.lm[h], ll = a.ll[h];
      float pmax = -INFINITY;
      for (int c = threadIdx.x; c < a.sc; c += blockDim.x)
        if (a.keep[(size_t)h * a.sc + c]) pmax = fmaxf(pmax, a.pm[(size_t)h * a.sc + c]);
      pmax = block_max(pmax, s.red);
      float ref = fmaxf(lm, pmax);
      float den = 0.f, wm = 0.f;
      for (int c = threadIdx.x; c < a.sc; c += blockDim.x)
        if (a.keep[(size_t)h * a.sc + c])
          den += wexp(a.pm[(size_t)h * a.sc + c], ref) * a.pl[(size_t)h * a.sc + c];
      for (int i = threadIdx.x; i < a.sp; i += blockDim.x)
        if (wrong[i]) wm += wexp(a.mass_m[(size_t)h * a.sp + i], ref) * a.mass_l[(size_t)h * a.sp + i];
      den = block_sum(den, s.red);
      wm = block_sum(wm, s.red);
      den += expf(lm - ref) * ll;
      extra = wm / den;
      skip = extra <= a.eps;
    }
    if (skip)
      for (int i = threadIdx.x; i < a.sp; i += blockDim.x) wrong[i] = 0;
    __syncthreads();
    int nneg = rank_flags(wrong, a.sp, rk, scan);
    for (int i = threadIdx.x; i < a.sp; i += blockDim.x)
      if (wrong[i]) store_id(a.queue, a.qtype, (int64_t)h * a.cap + nmiss + rk[i], s.p[i]);
    total += nneg;
    if (threadIdx.x == 0) a.low_hit[h] = lowhit;
  }
  if (threadIdx.x == 0) {
    a.pos[h] = nmiss;
    a.total[h] = total;
    if (a.eps > 0.f) {
      a.approx[h] = skip;
      a.extra[h] = skip ? extra : 0.f;
    }
  }
}

struct JobArgs {
  const void* q; const void* k; const void* v;
  int hq, hkv, n, b, d;
  const void* queue; int qtype; int cap;
  const int32_t* pos; const int32_t* total;
  const float* lm;
  int mode;
  int fused;   // 0: signed_repair partials, 1: signed_fused corrections
  float* m; float* l; float* u;
};

// One wave per (head, job).  Reference signed_repair.py:85-109 (block-local
// signed states) and signed_fused.py:30-67 (hybrid negatives computed
// block-locally then rescaled by exp(block_m - low_m); compact negatives
// evaluated directly in the low frame).
template <typename T, int VEC, int NC, int U>
__global__ __launch_bounds__(256) void k_jobs(JobArgs a) {
  using TL = Tile<T, VEC, NC>;
  int64_t item = (int64_t)blockIdx.x * kWaves + wave_id();
  if (item >= (int64_t)a.hq * a.cap) return;
  int h = (int)(item / a.cap);
  int job = (int)(item % a.cap);
  if (job >= a.total[h]) return;
  int64_t bid = load_id(a.queue, a.qtype, item);
  bool hybrid = a.mode != MODE_SAVED;
  bool negative = hybrid && job >= a.pos[h];
  TL t;
  t.init(a.d);
  float qr[TL::R];
  t.load_q(reinterpret_cast<const T*>(a.q) + (size_t)h * a.d, qr);
  int kv = h / (a.hq / a.hkv);
  float m = -INFINITY, l = 0.f, acc[TL::R];
#pragma unroll
  for (int i = 0; i < TL::R; ++i) acc[i] = 0.f;
  float store_m;
  if (bid >= 0 && bid < a.n) {
    size_t off = (((size_t)kv * a.n + bid) * a.b) * a.d;
    const T* kb = reinterpret_cast<const T*>(a.k) + off;
    const T* vb = reinterpret_cast<const T*>(a.v) + off;
    float scale = 1.0f / sqrtf((float)a.d);
    if (a.fused && a.mode == MODE_COMPACT && negative) {
      m = a.lm[h];
      t.template accum<U, true, true>(qr, kb, vb, a.b, scale, m, l, acc);
      t.finish(l, acc);
      store_m = m;
    } else {
      t.template accum<U, false, true>(qr, kb, vb, a.b, scale, m, l, acc);
      t.finish(l, acc);
      store_m = m;
      if (a.fused && a.mode == MODE_HYBRID && negative) {
        float target = a.lm[h];
        float f = expf(m - target);
        l *= f;
#pragma unroll
        for (int i = 0; i < TL::R; ++i) acc[i] *= f;
        store_m = target;
      }
    }
  } else {
    store_m = -INFINITY;
  }
  float sign = negative ? -1.f : 1.f;
  if (lane_id() == 0) {
    a.m[item] = store_m;
    a.l[item] = sign * l;
  }
  t.store(a.u + item * a.d, acc, sign);
}

struct FinalArgs {
  const void* q; const void* k; const void* v;
  int hq, hkv, n, b, d;
  const void* a; int atype; int sa;
  int sc, cap, mode, fused;
  const float* pm; const float* pl; const float* pu; const uint8_t* keep;
  const float* lm; const float* ll; const float* lu; const float* labs; const uint8_t* low_hit;
  const float* cm; const float* cl; const float* cu;
  const int32_t* pos; const int32_t* total;
  float min_remain, cancel, eps;
  float* out; uint8_t* bad; float* remain; uint8_t* approx; float* extra;
};

// signed_repair.py:112-172 (fused == 0, no inline fallback) and
// signed_fused.py:70-145 (fused == 1, inline strict fallback).
template <typename T, int VEC, int NC, int U>
__global__ __launch_bounds__(256) void k_finalize(FinalArgs a) {
  using TL = Tile<T, VEC, NC>;
  __shared__ HeadLds s;
  const int h = blockIdx.x;
  const int d = a.d;
  const bool hybrid = a.mode != MODE_SAVED;
  const int npos = a.pos[h], count = a.total[h];
  const float* pm = a.pm + (size_t)h * a.sc;
  const uint8_t* keep = a.keep + (size_t)h * a.sc;
  const float* cm = a.cm + (size_t)h * a.cap;
  const float* cl = a.cl + (size_t)h * a.cap;
  float pmax = -INFINITY, cmax = -INFINITY;
  for (int c = threadIdx.x; c < a.sc; c += blockDim.x) if (keep[c]) pmax = fmaxf(pmax, pm[c]);
  for (int j = threadIdx.x; j < npos; j += blockDim.x) cmax = fmaxf(cmax, cm[j]);
  pmax = block_max(pmax, s.red);
  cmax = block_max(cmax, s.red);
  float fraction = 1.f;
  bool bad = false;
  float low_m = -INFINITY, low_l = 0.f;
  bool lowhit = hybrid && a.low_hit[h];
  for (int dd = threadIdx.x; dd < d; dd += blockDim.x) s.u2[dd] = 0.f;   // low_u
  __syncthreads();
  if (lowhit) {
    low_m = a.lm[h];
    float ol = a.ll[h];
    // negatives: fused ones are already in the low frame; the 4-launch
    // states are block-local and rescaled by exp(cm - low_m)
    float dz = sum_states(
        s, count - npos, d,
        [&](int j) { return a.fused ? 1.f : wexp(cm[npos + j], low_m); },
        [&](int j) { return cl[npos + j]; },
        [&](int j) { return a.cu + ((size_t)h * a.cap + npos + j) * d; }, s.u1);
    low_l = ol + dz;
    fraction = low_l / ol;
    int cancel = 0;
    for (int dd = threadIdx.x; dd < d; dd += blockDim.x) {
      float du = s.u1[dd];
      float lu = a.lu[(size_t)h * d + dd] + du;
      s.u2[dd] = lu;
      float sc = a.labs[(size_t)h * d + dd] + fabsf(du);
      cancel |= (fabsf(lu) < a.cancel * sc) && (sc > 0.f);
    }
    cancel = block_or(cancel, s.ired);
    bad = (fraction < a.min_remain) || (fraction != fraction) || cancel;
  }
  float mx = fmaxf(fmaxf(pmax, cmax), low_m);
  float zp = sum_states(
      s, a.sc, d, [&](int c) { return keep[c] ? wexp(pm[c], mx) : 0.f; },
      [&](int c) { return a.pl[(size_t)h * a.sc + c]; },
      [&](int c) { return a.pu + ((size_t)h * a.sc + c) * d; }, s.u0);
  float zc = sum_states(
      s, npos, d, [&](int j) { return wexp(cm[j], mx); }, [&](int j) { return cl[j]; },
      [&](int j) { return a.cu + ((size_t)h * a.cap + j) * d; }, s.u1);
  float lw = wexp(low_m, mx);
  float z = zp + zc + lw * low_l;
  int invalid = 0;
  for (int dd = threadIdx.x; dd < d; dd += blockDim.x) {
    float num = s.u0[dd] + s.u1[dd] + lw * s.u2[dd];
    float o = num / z;
    s.u0[dd] = o;
    invalid |= is_bad(o);
  }
  invalid = block_or(invalid, s.ired);
  if (hybrid) bad = bad || invalid || (z <= 0.f) || (fabsf(z) == INFINITY);
  if (hybrid && bad && a.fused) {
    TL t;
    t.init(d);
    float qr[TL::R];
    t.load_q(reinterpret_cast<const T*>(a.q) + (size_t)h * d, qr);
    int kv = h / (a.hq / a.hkv);
    float mw, zw;
    stream_blocks<T, VEC, NC, U, false>(
        s, qr, t, (const T*)a.k, (const T*)a.v, kv, a.n, a.b, d, a.sa,
        [&](int j) -> int64_t { return load_id(a.a, a.atype, (int64_t)h * a.sa + j); }, 0.f, mw,
        zw, s.u1);
    for (int dd = threadIdx.x; dd < d; dd += blockDim.x) s.u0[dd] = s.u1[dd] / zw;
    __syncthreads();
  }
  for (int dd = threadIdx.x; dd < d; dd += blockDim.x) a.out[(size_t)h * d + dd] = s.u0[dd];
  if (threadIdx.x == 0) {
    a.bad[h] = bad;
    a.remain[h] = fraction;
    if (hybrid && bad && a.eps > 0.f) {
      a.approx[h] = 0;
      a.extra[h] = 0.f;
    }
  }
}

}  // namespace stk

using namespace stk;

extern "C" {

STK_API size_t stk_signed_workspace_bytes(int hq, int sa, int sp, int sc, int d, int mode) {
  int cap = mode == MODE_SAVED ? sa : sa + sp;
  return stk_align((size_t)hq * sc) + stk_align((size_t)hq) + stk_align((size_t)hq * cap * 4) * 2 +
         stk_align((size_t)hq * cap * d * 4);
}

// strict_topk/signed_repair.py:175-232 (fused == 0) and
// strict_topk/signed_fused.py:148-193 (fused == 1).  `queue` ([hq, cap],
// queue_dtype), `pos` and `total` ([hq] int32) are caller outputs.
STK_API int stk_repair_signed(const void* q, const void* k, const void* v, int dtype, int hq,
                              int hkv, int n, int b, int d, const void* selected, int sel_dtype,
                              int sa, const void* predicted, int pred_dtype, int sp, int mode,
                              int sc, const float* pm, const float* pl, const float* pu,
                              const uint8_t* high, const float* low_m, const float* low_l,
                              const float* low_u, const float* low_abs, const void* retained_ids,
                              const float* mass_m, const float* mass_l, float min_remaining,
                              float cancellation_tol, float max_extra_mass, int fused,
                              void* queue, int queue_dtype, int32_t* positive_jobs,
                              int32_t* total_jobs, float* out, uint8_t* fallback,
                              float* remaining, uint8_t* approximate, float* extra_mass_bound,
                              void* workspace, size_t workspace_bytes, void* stream) {
  STK_REQUIRE(stk_check_kv(dtype, hq, hkv, n, b, d));
  STK_REQUIRE(sa > 0 && sp > 0 && sa <= kMaxIds && sp <= kMaxIds, "ids must be nonempty (<= 4096)");
  STK_REQUIRE(mode >= 0 && mode <= 2, "bad prediction mode");
  STK_REQUIRE(q && k && v && selected && predicted && pm && pl && pu && queue && positive_jobs &&
                  total_jobs && out && fallback && remaining,
              "null pointer");
  STK_REQUIRE(mode == MODE_SAVED || (high && low_m && low_l && low_u && low_abs), "null low group");
  STK_REQUIRE(mode != MODE_COMPACT || retained_ids, "null retained ids");
  STK_REQUIRE(sc > 0 && sc <= kMaxIds, "bad prediction state width");
  STK_REQUIRE(max_extra_mass >= 0.f && max_extra_mass <= 1.f, "max_extra_mass must be in [0,1]");
  STK_REQUIRE(max_extra_mass == 0.f || (approximate && extra_mass_bound), "null budget outputs");
  STK_REQUIRE(max_extra_mass == 0.f || mode == MODE_SAVED || (mass_m && mass_l),
              "positive max_extra_mass requires speculate(..., keep_mass=True)");
  STK_REQUIRE(workspace && workspace_bytes >= stk_signed_workspace_bytes(hq, sa, sp, sc, d, mode),
              "workspace too small");
  hipStream_t st = (hipStream_t)stream;
  int cap = mode == MODE_SAVED ? sa : sa + sp;
  const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(pu);
  if (fused && mode != MODE_COMPACT && sc == sp && srepair_covers(dtype, b, d, sa, sp, align)) {
    // one launch: schedule, corrections and guarded merge (srepair.hip)
    SRepairArgs r{{q, k, v, hq, hkv, n, b, d}, selected, sel_dtype, sa, predicted, pred_dtype, sp,
                  mode == MODE_HYBRID ? 1 : 0, pm, pl, pu, high, low_m, low_l, low_u, low_abs,
                  mass_m, mass_l, min_remaining, cancellation_tol, max_extra_mass, queue,
                  queue_dtype, cap, positive_jobs, total_jobs, out, fallback, remaining,
                  approximate, extra_mass_bound};
    return launch_srepair(dtype, r, st);
  }
  Carve w(workspace);
  uint8_t* keep = w.take<uint8_t>((size_t)hq * sc);
  uint8_t* low_hit = w.take<uint8_t>((size_t)hq);
  float* cm = w.take<float>((size_t)hq * cap);
  float* cl = w.take<float>((size_t)hq * cap);
  float* cu = w.take<float>((size_t)hq * cap * d);
  SchedArgs sa_{selected, sel_dtype, sa, predicted, pred_dtype, sp, sc, mode, cap, high,
                retained_ids, pm, pl, low_m, low_l, mass_m, mass_l, max_extra_mass, queue,
                queue_dtype, positive_jobs, total_jobs, keep, low_hit, approximate,
                extra_mass_bound};
  hipLaunchKernelGGL(k_schedule, dim3(hq), dim3(256), 0, st, sa_);
  int rc = stk_check_launch("k_schedule");
  if (rc) return rc;
  JobArgs ja{q, k, v, hq, hkv, n, b, d, queue, queue_dtype, cap, positive_jobs, total_jobs, low_m,
             mode, fused ? 1 : 0, cm, cl, cu};
  int64_t items = (int64_t)hq * cap;
  int grid = (int)((items + kWaves - 1) / kWaves);
  STK_DISPATCH_TILE(dtype, d, {
    hipLaunchKernelGGL((k_jobs<T, VEC, NC, U>), dim3(grid), dim3(256), 0, st, ja);
  });
  rc = stk_check_launch("k_jobs");
  if (rc) return rc;
  FinalArgs fa{q, k, v, hq, hkv, n, b, d, selected, sel_dtype, sa, sc, cap, mode, fused ? 1 : 0,
               pm, pl, pu, keep, low_m, low_l, low_u, low_abs, low_hit, cm, cl, cu,
               positive_jobs, total_jobs, min_remaining, cancellation_tol, max_extra_mass, out,
               fallback, remaining, approximate, extra_mass_bound};
  STK_DISPATCH_TILE(dtype, d, {
    hipLaunchKernelGGL((k_finalize<T, VEC, NC, U>), dim3(hq), dim3(256), 0, st, fa);
  });
  rc = stk_check_launch("k_finalize");
  if (rc || fused || mode == MODE_SAVED) return rc;
  // 4-launch variant: separate strict fallback (kernels.py:223-247)
  return stk_fallback(q, k, v, dtype, hq, hkv, n, b, d, selected, sel_dtype, sa, fallback, out,
                      stream);
}

}  // extern "C"
