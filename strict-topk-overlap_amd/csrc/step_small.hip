// The speculative step for small shapes in one launch, one workgroup per
// query head and no hand-off between workgroups.
//
// The reference's step (benchmarks/run_benchmark.py:99-118, overlap_run:
// selector.select_blocks || kernels.speculate('saved'), joined, then
// kernels.repair or gqa.repair_union) is, per query head, the bound scores of
// its KV head's blocks (selector.py:8-20), their top-K, the predicted blocks'
// softmax states (kernels.py:42-71) and the strict repair's LSE merge
// (kernels.py:120-247).  When a head has at most 128 blocks and at most
// sixteen selected and sixteen predicted rows, one workgroup of sixteen waves
// holds all of it, in two roles that meet only in LDS:
//   * selection, waves 0..7 (launched first): wave 0 requests the predicted
//     IDs ahead of everything and publishes them as soon as they arrive;
//     every wave requests the bounds of N / 8 blocks (8 or 16) and the
//     query, scores them in FP64, publishes the keys, adds its partial ranks
//     (its blocks against all of them; past 64 blocks a lane ranks two), and
//     once every rank is in, each wave finds the selection and the misses by
//     ballot and requests its miss half-tiles (a miss is split in two
//     16-token halves, two per wave in flight, in one round up to eight
//     misses and two up to sixteen); wave 0 writes the IDs while those tiles
//     travel;
//   * prediction, waves 8..15: wave 8 + p waits for the IDs, then for slot
//     p and (past eight rows) slot p + 8 in turn requests the tile and
//     computes and stores its softmax state.
// The merge after the one barrier reads every row (predicted states, miss
// halves) from LDS.  Critical path: two dependent memory round trips (the
// bounds, then the miss tiles) and two LDS hand-offs (keys, ranks).  The
// one-launch step for larger shapes (k_step1) hands keys and states between
// workgroups through flags in memory, which costs more than the work here.
//
// Contracts as everywhere in the library: scores in FP64 in the fixed order
// (lane c of 16 sums dims 64 j + 4 c + t, j then t ascending, then the xor
// butterfly 8, 4, 2, 1; oracle bound_scores), keys order-preserving (NaN
// lowest), the top-K's ties toward the lower block index and IDs ascending;
// saved repair: a predicted slot counts when its block is selected and it is
// the highest slot holding that block; union: every predicted slot with a
// valid block; selected blocks in no predicted slot are computed from K/V.
#include "score.hpp"
#include "tile2.hpp"
#include "step_small.hpp"

namespace stk {

namespace {

// Intra-workgroup hand-offs between waves through LDS counters.  The fences
// order LDS only: a wave's global loads in flight (a tile it has requested)
// do not hold back its signal.  A waiting wave sleeps between its reads.
__device__ __forceinline__ void lds_signal(int* c) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  if (lane_id() == 0) __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_wait(int* c, int v) {
  while (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < v)
    __builtin_amdgcn_s_sleep(1);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// KB: blocks per lane of the rank (MAXN = 64 KB blocks per KV head at most);
// ROWS: the most selected and the most predicted rows per head (8 or 16).
template <typename T, int NCH, bool LB16, int KB, int ROWS>
__global__ __launch_bounds__(kSmallThreads) void k_step_small(SmallArgs a) {
  using TT = TokTile<T, NCH, 2>;   // 32 tokens: one block per chunk
  using TH = TokTile<T, NCH, 1>;   // 16 tokens: half a block (the misses)
  constexpr int D = TT::D;
  constexpr int P = D / 64;         // 64-dim scoring passes
  constexpr int SW = kSmallRoleWaves;
  constexpr int MAXN = STK_WAVE * KB;
  static_assert(KB == 1 || KB == 2, "one or two blocks per lane");
  constexpr int STEPS = MAXN / (SW * 4);         // 4-block scoring steps per wave
  constexpr int JW = MAXN / SW;                  // blocks per wave in the rank
  static_assert(ROWS == 8 || ROWS == 16, "eight or sixteen rows");
  constexpr int RM = 2 * ROWS;                   // the misses' half-block rows
  constexpr int R = ROWS + RM;                   // merged rows: predicted | miss halves
  constexpr int RC = 24;                         // rows per merge chunk
  static_assert(R % RC == 0 && RC % 8 == 0 && TH::QW == TT::QW && TH::DPL == TT::DPL,
                "rows merged in chunks of 24; the half tile shares the query layout");
  __shared__ uint64_t s_key[MAXN];
  __shared__ int s_rank[MAXN];
  __shared__ int s_pred[MAXN];   // 1: some predicted slot holds the block
  __shared__ int s_pid[ROWS];
  __shared__ __align__(16) int s_on[R];
  __shared__ int s_kdone, s_rdone, s_pdone;
  __shared__ __align__(16) float s_m[R];
  __shared__ __align__(16) float s_l[R];
  __shared__ __align__(16) float s_u[R][D];
  const int h = blockIdx.x, tid = threadIdx.x, w = wave_id(), lane = lane_id();
  const int n = a.n, sp = a.sp, K = a.k;
  const int kv = h / (a.hq / a.hkv);
  const T* K_ = reinterpret_cast<const T*>(a.kk);
  const T* V_ = reinterpret_cast<const T*>(a.vv);
  const size_t blk_elems = (size_t)32 * D;
  const T* qrow = reinterpret_cast<const T*>(a.q) + (size_t)h * D;
  const float scale = 1.0f / sqrtf((float)D);
  if (tid < MAXN) {
    s_rank[tid] = 0;
    s_pred[tid] = 0;
  }
  if (tid < R) s_on[tid] = 0;
  if (tid == 0) s_kdone = s_rdone = s_pdone = 0;
  __syncthreads();
  TT t;
  t.init();
  uint32_t qw[TT::QW];
  if (w >= SW) {
    // ---- predicted role, wave SW + q: slots q and (ROWS = 16) q + 8 in
    // turn, each its ID (published by wave 0), then its tile, then its state
    // (an invalid ID reads block 0 and keeps the empty state)
    if (w - SW < sp) {
      t.load_q(qrow, qw);
      lds_wait(&s_pdone, 1);
    }
    for (int ps = w - SW; ps < sp && ps < ROWS; ps += SW) {
      const int pid = s_pid[ps];
      const bool pvalid = pid >= 0;
      uint32_t kw[2][TT::QW], vw[TT::CH][TT::VW];
      const size_t off = ((size_t)kv * n + (pvalid ? pid : 0)) * blk_elems;
      t.load(K_ + off, V_ + off, 0, kw, vw);
      float m = -INFINITY, l = 0.f, acc[TT::DPL];
#pragma unroll
      for (int e = 0; e < TT::DPL; ++e) acc[e] = 0.f;
      if (pvalid) t.template update<false, false>(qw, kw, vw, 0, 32, scale, m, l, acc);
      const size_t row = (size_t)h * sp + ps;
      if (lane == 0) {
        a.m[row] = m;
        a.l[row] = l;
        s_m[ps] = m;
        s_l[ps] = l;
      }
      t.store(a.u + row * D, acc);
      t.store(s_u[ps], acc);
    }
  } else {
    // ---- selection role, wave sw: the bound scores of its blocks (every
    // load issued before any arithmetic).  Lane l16 of a 16-lane row is
    // logical lane c of the summation order (score_lane), so that the row
    // sum is DPP moves only
    const int sw = w;
    const int l16 = lane & 15, c = score_lane(l16), sub = lane >> 4;
    // wave 0 requests the predicted IDs first (the predicted role waits for
    // them; the bounds behind them take longer to arrive)
    int pidv = -1;
    if (sw == 0 && lane < sp) pidv = a.p[(size_t)h * sp + lane];
    uint2 q2[P];
#pragma unroll
    for (int j = 0; j < P; ++j) q2[j] = *reinterpret_cast<const uint2*>(qrow + 64 * j + 4 * c);
    using BV = std::conditional_t<LB16, uint2, float4>;
    BV lb[STEPS][P], hb[STEPS][P];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int nb = (s * SW + sw) * 4 + sub;
      const size_t row = ((size_t)kv * n + (nb < n ? nb : 0)) * D;
#pragma unroll
      for (int j = 0; j < P; ++j) {
        const size_t e = row + 64 * j + 4 * c;
        if constexpr (LB16) {
          lb[s][j] = *reinterpret_cast<const uint2*>(reinterpret_cast<const T*>(a.lo) + e);
          hb[s][j] = *reinterpret_cast<const uint2*>(reinterpret_cast<const T*>(a.hi) + e);
        } else {
          lb[s][j] = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.lo) + e);
          hb[s][j] = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.hi) + e);
        }
      }
    }
    t.load_q(qrow, qw);
    __builtin_amdgcn_sched_barrier(0);
    if (sw == 0) {
      const bool ok = lane < sp && pidv >= 0 && pidv < n;
      if (lane < ROWS) s_pid[lane] = ok ? pidv : -1;
      if (ok) s_pred[pidv] = 1;
      lds_signal(&s_pdone);
    }
    static_assert(STEPS == 2 || STEPS == 4, "two or four scoring steps");
    double acc[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      acc[s] = 0.0;
#pragma unroll
      for (int j = 0; j < P; ++j) {
        float qs[4], lv[4], hv[4];
        Unpack<T>::run(q2[j].x, qs);
        Unpack<T>::run(q2[j].y, qs + 2);
        if constexpr (LB16) {
          Unpack<T>::run(lb[s][j].x, lv);
          Unpack<T>::run(lb[s][j].y, lv + 2);
          Unpack<T>::run(hb[s][j].x, hv);
          Unpack<T>::run(hb[s][j].y, hv + 2);
        } else {
          lv[0] = lb[s][j].x; lv[1] = lb[s][j].y; lv[2] = lb[s][j].z; lv[3] = lb[s][j].w;
          hv[0] = hb[s][j].x; hv[1] = hb[s][j].y; hv[2] = hb[s][j].z; hv[3] = hb[s][j].w;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float b = qs[e] >= 0.f ? hv[e] : lv[e];   // lo where q < 0 or NaN
          acc[s] = fma((double)qs[e], (double)b, acc[s]);
        }
      }
    }
    // the xor butterfly 8, 4, 2, 1 of every step at once: row lane l16
    // holds step l16 / (16 / STEPS)'s sum.  Blocks past N get key 0, below
    // every score's key or equal to a NaN score's and at a higher index, so
    // they never outrank a block
    const double sum = score_rowsum<STEPS>(acc, l16);
    constexpr int LPS = 16 / STEPS;   // row lanes per step
    if ((l16 & (LPS - 1)) == 0) {
      const int nb = ((l16 / LPS) * SW + sw) * 4 + sub;
      s_key[nb] = nb < n ? score_key(sum) : 0ull;
    }
    lds_signal(&s_kdone);
    lds_wait(&s_kdone, SW);
    // ---- ranks by (key, -index): wave sw compares every block (lane i
    // holds blocks i and, KB = 2, i + 64) with blocks JW sw .. JW sw + JW - 1
    // and adds its counts
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int i = lane + STK_WAVE * kb;
      const uint64_t ki = s_key[i];
      int part = 0;
#pragma unroll
      for (int x = 0; x < JW; ++x) {
        const int j = sw * JW + x;
        const uint64_t kj = s_key[j];
        part += (kj > ki) || (kj == ki && j < i);
      }
      if (part) __hip_atomic_fetch_add(&s_rank[i], part, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    lds_signal(&s_rdone);
    lds_wait(&s_rdone, SW);
    // ---- every selection wave: the selection and the misses (selected, in
    // no predicted slot) in ascending order.  Miss i is two tasks, its
    // tokens 0..15 (task 2 i) and 16..31 (task 2 i + 1); wave sw takes tasks
    // sw + 16 r and sw + 16 r + 8 in round r, all of the same parity
    // (selm / mm word kb: blocks 64 kb .. 64 kb + 63)
    bool sel[KB];
    uint64_t selm[2] = {0ull, 0ull}, mm[2] = {0ull, 0ull};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int i = lane + STK_WAVE * kb;
      const int rk = s_rank[i], pr = s_pred[i];   // both read at once
      sel[kb] = (i < n) & (rk < K);
      selm[kb] = __ballot(sel[kb]);
      mm[kb] = __ballot(sel[kb] & (pr == 0));
    }
    const int nm0 = __popcll(mm[0]);
    const int nmiss = nm0 + __popcll(mm[1]);
    const int nt = 2 * nmiss;
    const int t0 = 16 * (sw & 1);
    // block of miss mi (ascending order): the mi-th set bit of mm
    auto miss_block = [&](int mi) {
      const int word = mi < nm0 ? 0 : 1;
      uint64_t x = mm[word];
      for (int i = word ? mi - nm0 : mi; i > 0; --i) x &= x - 1;
      return STK_WAVE * word + __builtin_ctzll(x);
    };
    TH th;
    th.init();
#pragma unroll
    for (int r = 0; r < ROWS / 8; ++r) {
      const int ta = sw + 2 * SW * r, tb = ta + SW;
      const bool has_a = ta < nt, has_b = tb < nt;
      uint32_t kwa[1][TH::QW], vwa[TH::CH][TH::VW], kwb[1][TH::QW], vwb[TH::CH][TH::VW];
      if (has_a) {
        const size_t off = ((size_t)kv * n + miss_block(ta >> 1)) * blk_elems;
        th.load(K_ + off, V_ + off, t0, kwa, vwa);
      }
      if (has_b) {
        const size_t off = ((size_t)kv * n + miss_block(tb >> 1)) * blk_elems;
        th.load(K_ + off, V_ + off, t0, kwb, vwb);
      }
      __builtin_amdgcn_sched_barrier(0);   // both halves requested before either is used
      if (r == 0 && sw == 0) {
        // while the tiles travel: the IDs out, and the rows the merge takes.
        // Predicted slot p counts when valid and (union, or its block is
        // selected and p is the highest slot holding it)
        const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
          if (sel[kb])
            a.ids[(size_t)h * K + (kb ? __popcll(selm[0]) : 0) + __popcll(selm[kb] & below)] =
                lane + STK_WAVE * kb;
        if (lane < sp) {
          const int b = s_pid[lane];
          bool top = true;
#pragma unroll
          for (int p = 0; p < ROWS; ++p)
            top = top && !(p > lane && p < sp && s_pid[p] == b);
          const bool bsel = b >= 0 && ((selm[b >> 6] >> (b & 63)) & 1ull);
          s_on[lane] = b >= 0 && (a.uni != 0 || (bsel && top));
        } else if (lane >= ROWS && lane < ROWS + nt) {
          s_on[lane] = 1;
        }
      }
      // the halves' states (row ROWS + task)
      if (has_a) {
        float m = -INFINITY, l = 0.f, acc[TH::DPL];
#pragma unroll
        for (int e = 0; e < TH::DPL; ++e) acc[e] = 0.f;
        th.template update<false, false>(qw, kwa, vwa, t0, 32, scale, m, l, acc);
        if (lane == 0) {
          s_m[ROWS + ta] = m;
          s_l[ROWS + ta] = l;
        }
        th.store(s_u[ROWS + ta], acc);
      }
      if (has_b) {
        float m = -INFINITY, l = 0.f, acc[TH::DPL];
#pragma unroll
        for (int e = 0; e < TH::DPL; ++e) acc[e] = 0.f;
        th.template update<false, false>(qw, kwb, vwb, t0, 32, scale, m, l, acc);
        if (lane == 0) {
          s_m[ROWS + tb] = m;
          s_l[ROWS + tb] = l;
        }
        th.store(s_u[ROWS + tb], acc);
      }
    }
  }
  __syncthreads();
  // ---- the LSE merge of the rows taken, by the selection role's first waves
  // (the predicted role's waves may still have global stores in flight).
  // Every row is read; rows not taken (LDS this launch never wrote) are left
  // out by selection, not by a zero weight
  const int dm = tid;
  if (dm < D) {
    // chunks of RC rows: their m, l and flags as 4-wide vectors and their u
    // column entries all requested before any is used
    auto chunk = [&](int c0, float (&mr)[RC], float (&lr)[RC], float (&ur)[RC], int (&on)[RC]) {
#pragma unroll
      for (int i = 0; i < RC / 4; ++i) {
        const float4 m4 = reinterpret_cast<const float4*>(s_m + c0)[i];
        const float4 l4 = reinterpret_cast<const float4*>(s_l + c0)[i];
        const int4 o4 = reinterpret_cast<const int4*>(s_on + c0)[i];
        mr[4 * i] = m4.x; mr[4 * i + 1] = m4.y; mr[4 * i + 2] = m4.z; mr[4 * i + 3] = m4.w;
        lr[4 * i] = l4.x; lr[4 * i + 1] = l4.y; lr[4 * i + 2] = l4.z; lr[4 * i + 3] = l4.w;
        on[4 * i] = o4.x; on[4 * i + 1] = o4.y; on[4 * i + 2] = o4.z; on[4 * i + 3] = o4.w;
      }
#pragma unroll
      for (int r = 0; r < RC; ++r) ur[r] = s_u[c0 + r][dm];
      hold_all(ur);
    };
    float mr[RC], ur[RC], lr[RC];
    int on[RC];
    float M = -INFINITY;
#pragma unroll
    for (int c0 = 0; c0 < R; c0 += RC) {
      if (R > RC || c0 == 0) chunk(c0, mr, lr, ur, on);
#pragma unroll
      for (int r = 0; r < RC; ++r) M = on[r] ? fmaxf(M, mr[r]) : M;
    }
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int c0 = 0; c0 < R; c0 += RC) {
      if (R > RC) chunk(c0, mr, lr, ur, on);   // one chunk: still in registers
#pragma unroll
      for (int r = 0; r < RC; ++r) {
        const float f = wexp(mr[r], M);
        num = on[r] ? num + f * ur[r] : num;
        den = on[r] ? den + f * lr[r] : den;
      }
    }
    a.out[(size_t)h * D + dm] = num / den;
  }
}

}  // namespace

bool small_covers(int dtype, int hq, int hkv, int n, int b, int d, int topk, int sp,
                  int bounds_dtype, uintptr_t align) {
  return (dtype == DT_BF16 || dtype == DT_F16) && hq % hkv == 0 && b == 32 &&
         (d == 64 || d == 128) && n >= 1 && n <= kSmallMaxN && topk >= 1 &&
         topk <= kSmallMaxRows && topk <= n && sp >= 1 && sp <= kSmallMaxRows &&
         stk_bounds_ok(dtype, bounds_dtype) && (align & 15) == 0;
}

int launch_small(int dtype, const SmallArgs& a, int bounds_dtype, hipStream_t st) {
  const dim3 grid(a.hq), block(kSmallThreads);
  const bool lb16 = bounds_dtype != 0;
#define STK_SMALL_R(T_, NCH_, KB_, R_)                                                       \
  do {                                                                                      \
    if (lb16) hipLaunchKernelGGL((k_step_small<T_, NCH_, true, KB_, R_>), grid, block, 0, st, a); \
    else hipLaunchKernelGGL((k_step_small<T_, NCH_, false, KB_, R_>), grid, block, 0, st, a);     \
  } while (0)
#define STK_SMALL_KB(T_, NCH_, KB_)                              \
  do {                                                           \
    if (a.k > 8 || a.sp > 8) STK_SMALL_R(T_, NCH_, KB_, 16);     \
    else STK_SMALL_R(T_, NCH_, KB_, 8);                          \
  } while (0)
#define STK_SMALL(T_, NCH_)                      \
  do {                                           \
    if (a.n > STK_WAVE) STK_SMALL_KB(T_, NCH_, 2); \
    else STK_SMALL_KB(T_, NCH_, 1);              \
  } while (0)
  if (dtype == DT_BF16) {
    if (a.d == 64) STK_SMALL(bf16s, 2);
    else STK_SMALL(bf16s, 4);
  } else {
    if (a.d == 64) STK_SMALL(f16s, 2);
    else STK_SMALL(f16s, 4);
  }
#undef STK_SMALL
#undef STK_SMALL_KB
#undef STK_SMALL_R
  return stk_check_launch("k_step_small");
}

}  // namespace stk
