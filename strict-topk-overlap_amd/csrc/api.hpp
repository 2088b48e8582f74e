// Host-side helpers shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

// The public declarations: every exported definition must match them.
#include "../../include/strict_topk.h"

#define STK_API __attribute__((visibility("default")))

void stk_set_error(const char* fmt, ...);
int stk_check_launch(const char* what);

struct StkCheck {
  bool ok;
  const char* msg;
};

// STK_REQUIRE(cond, msg) or STK_REQUIRE(StkCheck)
#define STK_REQUIRE_2(cond, msg)      \
  do {                                \
    if (!(cond)) {                    \
      stk_set_error("%s", msg);       \
      return STK_EINVAL;              \
    }                                 \
  } while (0)
#define STK_REQUIRE_1(chk)            \
  do {                                \
    StkCheck _c = (chk);              \
    if (!_c.ok) {                     \
      stk_set_error("%s", _c.msg);    \
      return STK_EINVAL;              \
    }                                 \
  } while (0)
#define STK_GET_MACRO(_1, _2, NAME, ...) NAME
#define STK_REQUIRE(...) STK_GET_MACRO(__VA_ARGS__, STK_REQUIRE_2, STK_REQUIRE_1)(__VA_ARGS__)

StkCheck stk_check_kv(int dtype, int hq, int hkv, int n, int b, int d);

inline size_t stk_align(size_t x) { return (x + 255) & ~(size_t)255; }

// Bump allocator over a caller-provided workspace (256-byte aligned pieces).
struct Carve {
  char* p;
  explicit Carve(void* base) : p(static_cast<char*>(base)) {}
  template <typename T>
  T* take(size_t count) {
    T* r = reinterpret_cast<T*>(p);
    p += stk_align(count * sizeof(T));
    return r;
  }
};

int stk_launch_states(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                      int n, int b, int d, const void* ids, int itype, int s,
                      const uint8_t* active, int active_kind, const void* pred, int ptype, int sp,
                      int32_t* slot, float* m, float* l, float* u, bool with_v, hipStream_t st);
// The KV group's query heads on the matrix cores (hier_mfma.hip): one merged
// state per (query head, four packs of 32 tokens) into m, l, u
// [hq, ceil(packs / 4)], or with blocks != 0 the block states [hq, s];
// bf16 / fp16, D = 128, B = 4 or 8, 8 <= hq / hkv <= 16, 16-byte aligned Q,
// K, V and u.
bool stk_hier_mfma_covers(int dtype, int hq, int hkv, int b, int d, uintptr_t align);
int stk_launch_hier_mfma(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                         int n, int b, int d, const void* ids, int itype, int s, float* m,
                         float* l, float* u, int blocks, hipStream_t st);
// Hierarchical exact / repair in one launch: one merged state per four packs
// of 32 / B positions ([hq, ceil(packs / 4)] into m, l, u); with slot_in, hits
// take the prediction's states (pm, pl, pu [hq, psp]).  Covers bf16 / fp16
// (and FP32) packed shapes (B = 4 or 8) with an even number of query heads
// per KV head.
bool stk_states_comb_covers(int dtype, int hq, int hkv, int b, int d, uintptr_t align);
int stk_launch_states_comb(const void* q, const void* k, const void* v, int dtype, int hq,
                           int hkv, int n, int b, int d, const void* ids, int itype, int s,
                           const int32_t* slot_in, int slot_shared, const float* pm,
                           const float* pl, const float* pu, int psp, float* m, float* l,
                           float* u, hipStream_t st);
int stk_launch_states_skip(const void* q, const void* k, const void* v, int dtype, int hq,
                           int hkv, int n, int b, int d, const void* ids, int itype, int s,
                           const int32_t* slot_in, int slot_shared, float* m, float* l, float* u,
                           hipStream_t st);
int stk_launch_merge(const float* m, const float* l, const float* u, const uint8_t* inc, int h,
                     int s, int d, float* out, hipStream_t st);

// lo / hi element type: STK_F32, or the keys' own 16-bit type (lb = 1).
inline bool stk_bounds_ok(int dtype, int bounds_dtype) {
  return bounds_dtype == 0 || (bounds_dtype == dtype && dtype != 0);
}

int stk_launch_score(const void* q, int q_dtype, const void* lo, const void* hi, int lb, int hq,
                     int hkv, int n, int d, float* scores, uint64_t* keys, hipStream_t st);
int stk_launch_topk(const uint64_t* keys, int rows, int n, int k, int32_t* ids, hipStream_t st);
