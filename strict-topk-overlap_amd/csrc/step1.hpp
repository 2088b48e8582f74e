// The speculative decode step in one launch.
//
// The reference's step (benchmarks/run_benchmark.py:99-118, overlap_run) is
// gqa.select_blocks || gqa.partials on the predicted blocks, joined, then
// the repair (gqa_light.repair_saved_light / gqa.repair_saved, or
// gqa.repair_union).  Here it is one grid of 512-thread workgroups in three
// roles, in launch order:
//   scoring   bound scores of a chunk of 64 blocks for every query head of a
//             KV head -> 64-bit top-K keys (score.hpp); then, once the
//             workgroup's stores have completed, one flag per (query head,
//             chunk);
//   states    one wave per (query head, predicted slot): the block's softmax
//             state (states_tok.hpp); then one flag per item;
//   tail      one workgroup per query head: waits for its chunk flags, runs
//             the exact top-K, requests its state flags while it lists the
//             misses, then issues the missed tiles with the state rows and
//             runs the saved / union repair and the merge (the arithmetic
//             of tail.hpp).
// The tails' top-K and miss tiles thus overlap the states' HBM traffic,
// instead of following it behind a kernel boundary.
//
// Coherence.  Keys and states are stored agent-coherent and read back with
// agent-coherent loads (st_agent / ld_agent, common.hpp); a flag is set only
// after the stores it covers have completed.  No cache-wide fence is used:
// an agent-scope release fence writes the whole L2 back, which measured about
// five times the step itself when every workgroup did it.
//
// Progress.  Producers never wait; the tails are the last workgroups of the
// grid, so every producer is dispatched no later than any tail, and 32-64
// waiting workgroups cannot fill a GPU.  Every wait is also bounded in time
// (kSpinTicks): past it the tail sets the error word and goes on.
//
// Flags.  A tail clears the flags it consumed before it ends, so the flag
// array is all zero between launches, whatever the shape: it must be zero
// before its first use and is then left so by every launch.
#pragma once

#include "step_launch.hpp"

namespace stk {

constexpr int kStep1Threads = kTailThreads;         // 512: eight waves per role
constexpr int kStep1Waves = kStep1Threads / STK_WAVE;
constexpr int kStep1Blocks = kStep1Waves * 4 * 2;   // blocks per scoring chunk

struct Step1Args {
  FrontArgs f;       // f.sc.sflag [hq, fstride], f.st.tflag [hq * sp]
  TailArgs t;
  uint32_t* err;     // counts timed-out waits
  uint64_t spin;     // longest wait, in ticks of the 100 MHz real-time counter
  int S, T, H;       // workgroups per role: scoring, states, tails
};

// The flag array's fewest words: one per (query head, chunk) and per (query
// head, slot).
inline size_t step1_ctl_words(int hq, int n, int sp) {
  const size_t chunks = ((size_t)n + kStep1Blocks - 1) / kStep1Blocks;
  return (size_t)hq * chunks + (size_t)hq * sp;
}

template <typename T, int NCH, int KPT, int RPT>
__device__ __forceinline__ void step1_tail(const Step1Args& A, int h) {
  const TailArgs& a = A.t;
  using TT = TokTile<T, NCH, 2>;
  constexpr int D = TT::D;
  constexpr int TPR = D / 4;              // threads per state row (16-byte columns)
  constexpr int RG = kTailThreads / TPR;  // rows per pass of the state loads
  // SP <= RG * RPT (the launch covers no more slots): two flags per lane
  static_assert(RG * RPT <= 2 * STK_WAVE, "the state flags are read two per lane");
  __shared__ int map[kTailMapN];
  __shared__ int sel[kTailMaxK], miss[kTailMaxK], pids[kTailMaxK];
  __shared__ TopkBinsLds tb;
  __shared__ int s_scan[kTailWaves];
  __shared__ int s_fail;   // a wave's wait timed out: the head's results are void
  __shared__ float s_hmax[kTailWaves], s_hl[kTailWaves];
  __shared__ __align__(16) float s_hu[kTailWaves][D];
  __shared__ float s_wm[kTailWaves], s_wl[kTailWaves], s_wu[kTailWaves][D];
  const int n = a.kv.n, sp = a.sp;
  const int tid = threadIdx.x, w = wave_id();
  const int G = a.kv.hq / a.kv.hkv;
  const int chunks = A.f.sc.chunks;
  uint32_t* sflag = A.f.sc.sflag + (size_t)h * A.f.sc.fstride;
  uint32_t* tflag = A.f.st.tflag + (size_t)h * sp;
  // ---- what depends on nothing: the predicted row and the query row
  const int pid = (int)ld_or(a.p, (int64_t)h * sp + tid, tid < sp, (int32_t)-1);
  TT t;
  t.init();
  uint32_t qw[TT::QW];
  t.load_q(reinterpret_cast<const T*>(a.kv.q) + (size_t)h * D, qw);
  for (int i = tid; i < n; i += kTailThreads) map[i] = 0;
  // the top-K's histogram too: it starts at phase B, with the row's range
  // from the scorers' flags
  for (int i = tid; i < kBins; i += kTailThreads) tb.hist[i] = 0;
  if (tid < kBins / 16) tb.grp[tid] = 0;
  if (tid == 0) tb.ncand = 0;
  // every slot entry is written (-1 past sp): the sums below read entries
  // past sp, and LDS holds whatever an earlier workgroup left there
  if (tid < kTailMaxK) pids[tid] = pid;
  if (tid == 0) s_fail = 0;
  __syncthreads();   // the clears before any use (the flags take far longer)
  // ---- this head's keys and their range, once every chunk of its KV head
  // is published.  Wave 0 polls the flags and the others wait at a barrier:
  // eight waves polling on their own phases would start the top-K with the
  // last of eight sightings
  __shared__ uint32_t s_rng[3];
  if (w == 0) {
    uint32_t mx, mn;
    const bool got = wait_flags_range(sflag, chunks, A.err, A.spin, mx, mn);
    if (lane_id() == 0) {
      s_rng[0] = mx;
      s_rng[1] = mn;
      s_rng[2] = got;
    }
  }
  __syncthreads();
  const uint32_t hmax = s_rng[0], hmin = s_rng[1];
  bool ok = s_rng[2] != 0u;
  uint64_t key[KPT];
  {
    const uint64_t* rk = a.keys + (size_t)h * n;
    const int base = tid * KPT;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const bool ok = base + i < n;
      const uint64_t x = ld_agent(rk + (ok ? base + i : 0));
      key[i] = ok ? x : 0ull;
    }
  }
  // membership map: max predicted slot + 1 of each valid predicted block (a
  // valid block always has a state here: the states role computes every slot)
  if (tid < sp && pid >= 0 && pid < n) atomicMax(&map[pid], tid + 1);
  const uint32_t flags = topk_bins_from<KPT>(key, n, a.k, tb, hmax, hmin);
  // ---- the state flags, requested now and read after the scan, so that
  // their round trip overlaps it (slots past SP read slot 0; SP <= 128 here)
  const int fl0 = lane_id(), fl1 = lane_id() + STK_WAVE;
  const uint32_t fv0 = ld_agent(tflag + (fl0 < sp ? fl0 : 0));
  const uint32_t fv1 = ld_agent(tflag + (fl1 < sp ? fl1 : 0));
  // ---- ranks of the selected IDs and the misses, one packed scan
  uint32_t mflags = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int idx = tid * KPT + i;
    const bool on = (flags >> i) & 1u;
    const int mv = map[on ? idx : 0];
    mflags |= (uint32_t)(on && mv == 0) << i;
  }
  int total;
  const int pre = block_excl_scan1(__popc(flags) | (__popc(mflags) << 16), s_scan, &total);
  int pos = pre & 0xffff, mpos = pre >> 16;
  const int nm = total >> 16;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int idx = tid * KPT + i;
    if ((flags >> i) & 1u) {
      sel[pos++] = idx;
      map[idx] |= kSelFlag;   // this thread's block: no other writer
    }
    if ((mflags >> i) & 1u) miss[mpos++] = idx;
  }
  __syncthreads();
  // ---- each wave's first missed tile (it needs no state), then every state
  // published, then the state rows.  Checking the flag values requested
  // before the scan waits for them only (loads return in order, and the
  // tile's went out after them); only the rare wait for the last flags also
  // waits behind the tile
  const int kvh = h / G;
  const float scale = 1.0f / sqrtf((float)D);
  const T* K = reinterpret_cast<const T*>(a.kv.k);
  const T* V = reinterpret_cast<const T*>(a.kv.v);
  auto tile = [&](int x) { return (((size_t)kvh * n + miss[x]) * a.kv.b) * D; };
  uint32_t kw[2][TT::QW], vw[TT::CH][TT::VW];
  if (w < nm) t.load(K + tile(w), V + tile(w), 0, kw, vw);
  if (!__all((fv0 != 0u || fl0 >= sp) && (fv1 != 0u || fl1 >= sp)))
    ok = wait_flags(tflag, sp, A.err, A.spin) && ok;
  // ---- this head's prediction states (thread (rg, c4): columns 4 c4 .. +3
  // of rows rg + RG j)
  const int c4 = tid % TPR, rg = tid / TPR;
  float um[RPT], ul[RPT];
  float4 uu[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int r = rg + RG * j;
    const int64_t row = (int64_t)h * sp + (r < sp ? r : 0);
    um[j] = ld_agentf(a.pm + row);
    ul[j] = ld_agentf(a.pl + row);
    const uint64_t* up = reinterpret_cast<const uint64_t*>(a.pu + row * D + 4 * c4);
    const uint64_t x0 = ld_agent(up), x1 = ld_agent(up + 1);
    uu[j] = make_float4(__uint_as_float((uint32_t)x0), __uint_as_float((uint32_t)(x0 >> 32)),
                        __uint_as_float((uint32_t)x1), __uint_as_float((uint32_t)(x1 >> 32)));
  }
  // ---- the first missed tile's state with the online softmax (the state
  // rows travel meanwhile)
  float m = -INFINITY, l = 0.f, acc[TT::DPL];
#pragma unroll
  for (int e = 0; e < TT::DPL; ++e) acc[e] = 0.f;
  if (w < nm) t.template update<false, false>(qw, kw, vw, 0, a.kv.b, scale, m, l, acc);
  // ---- the hits' (union: every valid predicted row's) partial LSE sums:
  // saved mode takes slot p when P[p] is selected and p is the highest slot
  // holding that block
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
    const int mv = map[pv[j] < 0 ? 0 : (pv[j] > nlast ? nlast : pv[j])];
    const bool hit = ((mv & kSelFlag) != 0) & ((mv & ~kSelFlag) == r + 1);
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
  // ---- a wave's further misses (more than eight per head), once the state
  // rows' registers are free (holding both would spill registers)
  for (int x = w + kTailWaves; x < nm; x += kTailWaves) {
    t.load(K + tile(x), V + tile(x), 0, kw, vw);
    t.template update<false, false>(qw, kw, vw, 0, a.kv.b, scale, m, l, acc);
  }
  if (lane_id() == 0) {
    s_wm[w] = m;
    s_wl[w] = l;
  }
  t.store(s_wu[w], acc);
  if (!ok && lane_id() == 0) atomicOr(&s_fail, 1);
  __syncthreads();
  // a timed-out wait read keys or states that may not have been published:
  // the head's output is NaN and its IDs -1, so the failure cannot pass for a
  // result (stk_step1_timeouts counts it)
  const bool fail = s_fail != 0;
  // ---- every wave is past its waits: clear this head's flags for the next
  // launch (no producer writes them again in this one)
  if (tid < chunks) st_agent(sflag + tid, 0u);
  if (tid < sp) st_agent(tflag + tid, 0u);
  // ---- one LSE merge of the hits' partials and the waves' miss states
  if (tid < D) {
    // every LDS value the merge reads is requested before any is used
    float hm[kTailWaves], wm[kTailWaves], hl[kTailWaves], wl[kTailWaves];
    float hu[kTailWaves], wu[kTailWaves];
#pragma unroll
    for (int x = 0; x < kTailWaves; ++x) {
      hm[x] = s_hmax[x];
      wm[x] = s_wm[x];
      hl[x] = s_hl[x];
      wl[x] = s_wl[x];
      hu[x] = s_hu[x][tid];
      wu[x] = s_wu[x][tid];
    }
    hold_all(hu);
    hold_all(wu);
    float M = -INFINITY;
#pragma unroll
    for (int x = 0; x < kTailWaves; ++x) M = fmaxf(M, fmaxf(hm[x], wm[x]));
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int x = 0; x < kTailWaves; ++x) {
      const float fh = wexp(hm[x], M), f = wexp(wm[x], M);
      num += fh * hu[x] + f * wu[x];
      den += fh * hl[x] + f * wl[x];
    }
    a.out[(size_t)h * D + tid] = fail ? __builtin_nanf("") : num / den;
  }
  // the selected IDs last (stores share the loads' counter: issued earlier,
  // they would hold the waits above)
  for (int i = tid; i < a.k; i += kTailThreads) a.ids[(size_t)h * a.k + i] = fail ? -1 : sel[i];
}

// T: bf16 / fp16; NCH: D / 32 (D = 64 or 128); blocks of 32 tokens; up to
// four query heads per KV head (the scorer stages them in one pass).
template <typename T, int NCH, int KPT, int RPT>
__global__ __launch_bounds__(kStep1Threads, 4) void k_step1(Step1Args a) {
  constexpr int P = NCH / 2;   // 64-dim passes of the scorer
  // Wave priorities (s_setprio: instruction arbitration inside a CU only):
  // the scorers' arithmetic, which the tails' keys wait on, and then the
  // tails' chain go ahead of co-resident states waves (measured: about
  // 0.05 us less per c3 step at 90 and 100 % overlap, no change at 75 %).
  const int b = blockIdx.x;
  if (b < a.S) {
    __builtin_amdgcn_s_setprio(3);
    score_wg<T, P, 2, true, 4, false, true, kStep1Waves>(a.f.sc, xcd_remap(b, a.S));
  } else if (b < a.S + a.T) {
    states_tok_wg<T, NCH, 2, int32_t, true, false, true>(a.f.st, xcd_remap(b - a.S, a.T));
  } else {
    __builtin_amdgcn_s_setprio(2);
    step1_tail<T, NCH, KPT, RPT>(a, xcd_remap(b - a.S - a.T, a.H));
  }
}

// True when k_step1 covers a fused-step shape (bf16 / fp16, B = 32, D in
// {64, 128}, at most four query heads per KV head, SP * D <= 8192: four
// state rows per thread of the tail).
bool step1_covers(int dtype, int hq, int hkv, int b, int d, const StepShape& s);

// Launch k_step1 when step1_covers the shape (returns 1 otherwise, with
// nothing launched).  ctl: `cap` >= step1_ctl_words(hq, n, sp) zero words
// (left zero; when they fit, each head's chunk flags start a 128-byte line of
// their own, so that no two heads' pollers share one); err: a word incremented for every timed-out wait; spin: the longest
// wait in ticks; drop (tests only): the producers publish no flag, so every
// wait times out.
int launch_step1(int dtype, const FrontArgs& f, const TailArgs& t, const StepShape& s,
                 uint32_t* ctl, size_t cap, uint32_t* err, uint64_t spin, int drop,
                 hipStream_t st);

}  // namespace stk
