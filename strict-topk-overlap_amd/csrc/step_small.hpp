// The speculative step for small shapes in one launch (k_step_small,
// step_small.hip): one workgroup per query head for up to 128 blocks per KV
// head and up to sixteen selected and sixteen predicted rows per head.  Its
// sixteen waves split in two roles (step_small.hip).
#pragma once

#include "api.hpp"

namespace stk {

constexpr int kSmallThreads = 1024;
constexpr int kSmallRoleWaves = 8;   // waves per role: predicted tiles | selection and misses
constexpr int kSmallMaxN = 128;     // blocks per KV head: up to two per lane of the rank
constexpr int kSmallMaxRows = 16;   // selected and predicted rows: up to two tiles per wave each

struct SmallArgs {
  const void* q; const void* kk; const void* vv;   // q [hq, d], k / v [hkv, n, 32, d]
  const void* lo; const void* hi;                  // [hkv, n, d], FP32 or q's type
  int hq, hkv, n, d;
  const int32_t* p; int sp;                        // predicted [hq, sp]
  int k;                                           // selected per head
  int uni;                                         // 1: repair_union
  int32_t* ids;                                    // [hq, k]
  float* m; float* l; float* u;                    // prediction states [hq, sp(, d)]
  float* out;                                      // [hq, d]
};

// True when k_step_small covers the fused step's shape: bf16 / fp16 K/V,
// B = 32, D in {64, 128}, N <= 128, TOPK and SP in [1, 16], bounds FP32 or of
// the K/V type, and 16-byte aligned q / k / v / lo / hi (`align`: the OR of
// their addresses).
bool small_covers(int dtype, int hq, int hkv, int n, int b, int d, int topk, int sp,
                  int bounds_dtype, uintptr_t align);

int launch_small(int dtype, const SmallArgs& a, int bounds_dtype, hipStream_t st);

}  // namespace stk
