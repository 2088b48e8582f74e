// Kernels of the fused decode steps and their shape dispatch, templated on
// PG (paged, batched KV).  step.hip and sstep.hip instantiate the dense
// kernels (PG = false), paged.hip the paged ones, so every kernel is built
// in exactly one translation unit.
//   k_front   one grid whose workgroups are either scoring workgroups (bound
//             score of a chunk of blocks -> 64-bit keys) or speculation
//             workgroups (per-block softmax states of the predicted blocks,
//             one wave per (query head, slot)), the two roles interleaved
//             evenly inside every XCD so both streams of HBM traffic run side
//             by side on all of them;
//   k_tail    one workgroup per query head: exact top-K, then the saved /
//             union repair (tail.hpp);
//   k_stail   one workgroup per query head: exact top-K, then the hybrid
//             grouping, signed corrections and guarded merge
//             (tail_signed.hpp).
#pragma once

#include "step.hpp"
#include "tail.hpp"
#include "tail_signed.hpp"

namespace stk {

template <typename T, int NCH, int UP, bool ONE, int P, int STEPS, int GT, bool PG>
__global__ __launch_bounds__(256, NCH <= 4 ? 4 : 2) void k_front(FrontArgs a) {
  // Workgroups are dealt round-robin over the 8 XCDs; roles are interleaved
  // on an XCD-contiguous logical index, so every XCD gets an even mix of
  // scoring and speculation work (and, with G query heads per KV head, the
  // scoring and the states of one KV head land on the same XCD's L2).
  const int i = xcd_remap(blockIdx.x, gridDim.x);
  // score workgroups among logical indices [0, i) and [0, i]
  const int before = (int)(((int64_t)i * a.score_wgs) / a.total_wgs);
  const int upto = (int)(((int64_t)(i + 1) * a.score_wgs) / a.total_wgs);
  if (upto > before)
    score_wg<T, P, STEPS, true, GT, PG>(a.sc, before, a.pg);
  else
    states_tok_wg<T, NCH, UP, int32_t, ONE, PG>(a.st, i - upto, a.pg);
}

template <typename T, int NCH, int UP, bool ONE, int KPT, int RPT, bool PG>
__global__ __launch_bounds__(kTailThreads) void k_tail(TailArgs a) {
  tail_head<T, NCH, UP, ONE, KPT, RPT, PG>(a);
}

template <typename T, int NCH, int UP, bool ONE, int KPT, int RPT, bool PG>
__global__ __launch_bounds__(kTailThreads) void k_stail(STailArgs a) {
  stail_head<T, NCH, UP, ONE, KPT, RPT, PG>(a);
}

namespace launch {

template <bool PG, typename T, int NCH, int UP, bool ONE, int P, int STEPS>
int front_gt(const FrontArgs& f, const StepShape& s, hipStream_t st) {
  const dim3 grid(f.total_wgs), block(256);
  if (s.gt == 1)
    hipLaunchKernelGGL((k_front<T, NCH, UP, ONE, P, STEPS, 1, PG>), grid, block, 0, st, f);
  else if (s.gt == 2)
    hipLaunchKernelGGL((k_front<T, NCH, UP, ONE, P, STEPS, 2, PG>), grid, block, 0, st, f);
  else
    hipLaunchKernelGGL((k_front<T, NCH, UP, ONE, P, STEPS, 4, PG>), grid, block, 0, st, f);
  return stk_check_launch("k_front");
}

template <bool PG, typename T, int NCH>
int front_t(const FrontArgs& f, const StepShape& s, hipStream_t st) {
  constexpr int P = NCH * 16 / (int)sizeof(T) * 4 / 64;   // D / 64
  constexpr int STEPS = P <= 2 ? 2 : 1;
  // ONE: the whole block is one token chunk (B == 16 * UP)
  return s.up == 1 ? (s.one ? front_gt<PG, T, NCH, 1, true, P, STEPS>(f, s, st)
                            : front_gt<PG, T, NCH, 1, false, P, STEPS>(f, s, st))
                   : (s.one ? front_gt<PG, T, NCH, 2, true, P, STEPS>(f, s, st)
                            : front_gt<PG, T, NCH, 2, false, P, STEPS>(f, s, st));
}

template <bool PG>
int front(int dtype, const FrontArgs& f, const StepShape& s, hipStream_t st) {
  if (f.total_wgs == 0) return STK_OK;
  STK_DISPATCH_STEP(dtype, s.nch, { return front_t<PG, T, NCH>(f, s, st); });
  return STK_EINVAL;
}

template <bool PG, typename T, int NCH, int UP, bool ONE>
int tail_one(const TailArgs& t, const StepShape& s, hipStream_t st) {
  const dim3 grid(t.kv.hq), block(kTailThreads);
#define STK_TAIL(KPT)                                                                   \
  if (s.rpt == 4)                                                                       \
    hipLaunchKernelGGL((k_tail<T, NCH, UP, ONE, KPT, 4, PG>), grid, block, 0, st, t);   \
  else                                                                                  \
    hipLaunchKernelGGL((k_tail<T, NCH, UP, ONE, KPT, 16, PG>), grid, block, 0, st, t);
  if (s.kpt == 4) { STK_TAIL(4) }
  else if (s.kpt == 8) { STK_TAIL(8) }
  else { STK_TAIL(16) }
#undef STK_TAIL
  return stk_check_launch("k_tail");
}

template <bool PG>
int tail(int dtype, const TailArgs& t, const StepShape& s, hipStream_t st) {
  STK_DISPATCH_STEP(dtype, s.nch, {
    return s.up == 1 ? (s.one ? tail_one<PG, T, NCH, 1, true>(t, s, st)
                              : tail_one<PG, T, NCH, 1, false>(t, s, st))
                     : (s.one ? tail_one<PG, T, NCH, 2, true>(t, s, st)
                              : tail_one<PG, T, NCH, 2, false>(t, s, st));
  });
  return STK_EINVAL;
}

template <bool PG, typename T, int NCH, int UP, bool ONE>
int stail_one(const STailArgs& t, const StepShape& s, hipStream_t st) {
  const dim3 grid(t.kv.hq), block(kTailThreads);
#define STK_STAIL(KPT)                                                                  \
  if (s.rpt == 4)                                                                       \
    hipLaunchKernelGGL((k_stail<T, NCH, UP, ONE, KPT, 4, PG>), grid, block, 0, st, t);  \
  else                                                                                  \
    hipLaunchKernelGGL((k_stail<T, NCH, UP, ONE, KPT, 16, PG>), grid, block, 0, st, t);
  if (s.kpt == 4) { STK_STAIL(4) }
  else if (s.kpt == 8) { STK_STAIL(8) }
  else { STK_STAIL(16) }
#undef STK_STAIL
  return stk_check_launch("k_stail");
}

template <bool PG>
int stail(int dtype, const STailArgs& t, const StepShape& s, hipStream_t st) {
  STK_DISPATCH_STEP(dtype, s.nch, {
    return s.up == 1 ? (s.one ? stail_one<PG, T, NCH, 1, true>(t, s, st)
                              : stail_one<PG, T, NCH, 1, false>(t, s, st))
                     : (s.one ? stail_one<PG, T, NCH, 2, true>(t, s, st)
                              : stail_one<PG, T, NCH, 2, false>(t, s, st));
  });
  return STK_EINVAL;
}

}  // namespace launch

// Each instantiation set lives in one translation unit of its own (the
// kernels are large and compile in parallel): launch_front (step.hip),
// launch_tail (tail_dense.hip), launch_stail (sstep.hip) and their paged
// counterparts (front_pg.hip, tail_pg.hip, stail_pg.hip).
int launch_tail(int dtype, const TailArgs& t, const StepShape& s, hipStream_t st);
int launch_front_pg(int dtype, const FrontArgs& f, const StepShape& s, hipStream_t st);
int launch_tail_pg(int dtype, const TailArgs& t, const StepShape& s, hipStream_t st);
int launch_stail_pg(int dtype, const STailArgs& t, const StepShape& s, hipStream_t st);
}  // namespace stk
