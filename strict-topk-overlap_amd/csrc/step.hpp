// The front of the fused decode steps, shared by the saved/union step
// (step.hip) and the signed step (sstep.hip): one grid that scores every
// block into 64-bit top-K keys while other workgroups compute the predicted
// blocks' softmax states.
#pragma once

#include "score.hpp"
#include "states_tok.hpp"
#include "api.hpp"

namespace stk {

struct FrontArgs {
  ScoreArgs sc;
  StatesArgs st;
  int score_wgs, total_wgs;
  Paging pg;             // paged, batched KV (the PG kernels only)
};

// Compile-time shape choices of one fused step.
struct StepShape {
  int nch, passes, steps, gt, kpt, up, rpt;
  bool one;
};

// Shape plan of a fused step, or a message saying why it is not supported.
const char* plan_step(int dtype, int hq, int hkv, int n, int b, int d, int topk, int sp,
                      int pred_dtype, uintptr_t align, StepShape* s);

// Front arguments: keys[hq, n] into `keys`, states of predicted[hq, sp]
// into m, l, u; lb: lo / hi are 16-bit (the element type of q, k, v).
FrontArgs make_front_args(const void* q, const void* k, const void* v, int dtype, int hq,
                          int hkv, int n, int b, int d, const void* lo, const void* hi, int lb,
                          const void* predicted, int sp, float* m, float* l, float* u,
                          uint64_t* keys, const StepShape& s);

// Launch k_front for (dtype, shape) on `st`.
int launch_front(int dtype, const FrontArgs& f, const StepShape& s, hipStream_t st);

}  // namespace stk

// Dispatch over the fused steps' element types (bf16, fp16) and token-tile
// widths (NCH 16-byte chunks per lane).
#define STK_DISPATCH_STEP(dtype, nch, ...)                        \
  do {                                                            \
    if (dtype == stk::DT_BF16) {                                  \
      using T = stk::bf16s;                                       \
      if (nch == 2) { constexpr int NCH = 2; __VA_ARGS__; }       \
      else if (nch == 4) { constexpr int NCH = 4; __VA_ARGS__; }  \
      else { constexpr int NCH = 8; __VA_ARGS__; }                \
    } else {                                                      \
      using T = stk::f16s;                                        \
      if (nch == 2) { constexpr int NCH = 2; __VA_ARGS__; }       \
      else if (nch == 4) { constexpr int NCH = 4; __VA_ARGS__; }  \
      else { constexpr int NCH = 8; __VA_ARGS__; }                \
    }                                                             \
  } while (0)
