// The signed repair with inline fallback in one launch (the drop-in
// repair_signed_fused for saved and hybrid predictions).
#pragma once

#include "common.hpp"

namespace stk {

struct SRepairArgs {
  KV kv;                                   // q, k, v, hq, hkv, n, b, d
  const void* a; int atype; int sa;        // selected [hq, sa]
  const void* p; int ptype; int sp;        // predicted [hq, sp]
  int hybrid;                              // 1: hybrid prediction, 0: saved
  const float* pm; const float* pl; const float* pu;   // prediction states [hq, sp(, d)]
  const uint8_t* high;                     // [hq, sp] (hybrid)
  const float* lm; const float* ll;        // low group [hq] (hybrid)
  const float* lu; const float* labs;      // [hq, d] (hybrid)
  const float* mass_m; const float* mass_l;   // [hq, sp] (eps > 0)
  float min_remain, cancel, eps;
  void* queue; int qtype; int cap;         // [hq, cap] job queue out
  int32_t* pos; int32_t* total;            // [hq] job counts out
  float* out; uint8_t* bad; float* remain; // [hq, d], [hq], [hq]
  uint8_t* approx; float* extra;           // [hq] when eps > 0
};

// Whether the one-launch kernel covers the shape: bf16 / fp16, D in
// {64, 128, 256}, B a multiple of 16, SA and SP <= 256, SP * D <= 32768,
// 16-byte aligned q / k / v / state rows.
bool srepair_covers(int dtype, int b, int d, int sa, int sp, uintptr_t align);

int launch_srepair(int dtype, const SRepairArgs& a, hipStream_t st);

}  // namespace stk
