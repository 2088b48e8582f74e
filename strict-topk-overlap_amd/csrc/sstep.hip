// The signed speculative decode step in two launches on one stream: the
// fused step's front (bound scores -> 64-bit keys || predicted-block
// states), then k_stail, one workgroup per query head doing the top-K, the
// hybrid grouping, the signed corrections and the guarded merge with the
// strict fallback (tail_signed.hpp).
//
// The reference composes this step as overlap_run(select_blocks,
// speculate(mode, keep_mass=True)) followed by repair_signed_fused
// (benchmarks/run_benchmark.py:99-118, strict_topk/signed_fused.py:148-193):
// nine launches on two streams.
#include "step_launch.hpp"

using namespace stk;

extern "C" {

STK_API int stk_signed_step(const void* q, const void* k, const void* v, int dtype, int hq,
                            int hkv, int n, int b, int d, const void* lo, const void* hi,
                            int bounds_dtype, int topk, const void* predicted, int pred_dtype, int sp, int hybrid,
                            float mass_threshold, float min_remaining, float cancellation_tol,
                            float max_extra_mass, int32_t* selected, float* m, float* l, float* u,
                            float* out, uint8_t* fallback, float* remaining, uint8_t* approx,
                            float* extra, int32_t* positive, int32_t* total, void* workspace,
                            size_t workspace_bytes, void* stream) {
  STK_REQUIRE(stk_check_kv(dtype, hq, hkv, n, b, d));
  STK_REQUIRE(q && k && v && lo && hi && predicted && selected && m && l && u && out &&
                  fallback && remaining && positive && total,
              "null pointer");
  STK_REQUIRE(stk_bounds_ok(dtype, bounds_dtype),
              "lo and hi must be FP32 or the element type of Q/K/V");
  STK_REQUIRE(!(max_extra_mass > 0.f) || (approx && extra),
              "max_extra_mass > 0 needs the approx and extra outputs");
  STK_REQUIRE(max_extra_mass >= 0.f && max_extra_mass <= 1.f, "max_extra_mass must be in [0,1]");
  STK_REQUIRE(mass_threshold >= 0.f && mass_threshold <= 1.f,
              "mass_threshold must be in [0,1]");
  STK_REQUIRE(workspace && workspace_bytes >= stk_step_workspace_bytes(hq, hkv, n, d, topk),
              "workspace too small");
  const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(u) |
                          reinterpret_cast<uintptr_t>(lo) | reinterpret_cast<uintptr_t>(hi);
  StepShape s{};
  const char* why = plan_step(dtype, hq, hkv, n, b, d, topk, sp, pred_dtype, align, &s);
  STK_REQUIRE(why == nullptr, why ? why : "");
  uint64_t* keys = static_cast<uint64_t*>(workspace);
  const FrontArgs f = make_front_args(q, k, v, dtype, hq, hkv, n, b, d, lo, hi,
                                      bounds_dtype != 0, predicted, sp, m, l, u, keys, s);
  STailArgs t{};
  t.kv = KV{q, k, v, hq, hkv, n, b, d};
  t.keys = keys; t.k = topk; t.ids = selected;
  t.p = static_cast<const int32_t*>(predicted); t.sp = sp;
  t.pm = m; t.pl = l; t.pu = u;
  t.hybrid = hybrid ? 1 : 0;
  t.tau = mass_threshold; t.min_remaining = min_remaining; t.cancel_tol = cancellation_tol;
  t.eps = max_extra_mass;
  t.out = out; t.bad = fallback; t.remain = remaining;
  t.approx = max_extra_mass > 0.f ? approx : nullptr;
  t.extra = max_extra_mass > 0.f ? extra : nullptr;
  t.pos = positive; t.total = total;
  hipStream_t st = (hipStream_t)stream;
  const int rc = launch_front(dtype, f, s, st);
  if (rc) return rc;
  return launch::stail<false>(dtype, t, s, st);
}

}  // extern "C"
