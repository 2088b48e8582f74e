// Paged, ragged KV and batched fused decode steps.
//
// A batch of R requests runs as one step: one k_front grid over every
// request's blocks and predicted slots, then one tail workgroup per
// (request, query head).  K/V live in a page pool [P, B, D] (one page = one
// KV head's block of B tokens), the block bounds in lo/hi pages [P, D], and
// block_table[r, kvh, j] names the page of logical block j of (request r,
// KV head kvh) for j < nblocks[r]; ntokens[r] (optional) is the request's
// token count, so its last block may be partly filled (tokens past the count
// get no weight).  The batch is flattened into R * Hq query
// heads over R * Hkv KV rows, so the kernels are the dense step's with the
// page indirection compiled in (PG = true): a page index is validated before
// every use, and an invalid one contributes the empty state.
//
// Reference: the reference reaches a paged cache only through FlashInfer's
// page table (strict_topk/flashinfer_backend.py:35-40, page = block +
// kv_head * N over k.view(hkv * n, b, 1, d), one request per call).  Per
// request, the results are those of the dense fused steps (stk_speculative_step,
// stk_signed_step) on the request's blocks gathered from the pool, bit for
// bit; a request with fewer blocks than K selects all of them.
#include "step_launch.hpp"

using namespace stk;

namespace {

constexpr size_t kPgDummy = 4096;   // stands in for absent predicted rows (sp == 0)

struct PagedPlan {
  StepShape s;
  int hq, hkv;      // flattened over the batch
};

StkCheck check_paged(int dtype, int requests, int hq, int hkv, int nb, int b, int d, int pages,
                     int topk, int sp) {
  if (requests < 1) return {false, "expected at least one request"};
  StkCheck c = stk_check_kv(dtype, hq, hkv, nb, b, d);
  if (!c.ok) return c;
  if (hq < 1) return {false, "expected nonempty shapes"};
  if (pages < 1) return {false, "the page pool is empty"};
  if (topk < 1 || topk > kTailMaxK) return {false, "topk must be in [1, 256]"};
  if (sp < 0 || sp > kTailMaxK) return {false, "the predicted width must be in [0, 256]"};
  if ((int64_t)requests * hq > 0x7fffffff / 8 || (int64_t)requests * hkv * nb > 0x7fffffff)
    return {false, "batch too large"};
  return {true, ""};
}

}  // namespace

extern "C" {

STK_API size_t stk_paged_workspace_bytes(int requests, int hq, int nb) {
  if (requests <= 0 || hq <= 0 || nb <= 0) return 0;
  return stk_align((size_t)requests * hq * nb * sizeof(uint64_t)) + kPgDummy;
}

static int paged_common(const void* q, const void* k_pages, const void* v_pages, int dtype,
                        int requests, int hq, int hkv, int nb, int b, int d, int pages,
                        const void* lo_pages, const void* hi_pages, int bounds_dtype,
                        const int32_t* table,
                        const int32_t* nblocks, const int32_t* ntokens, int topk,
                        const int32_t* predicted, int sp, float* m, float* l, float* u,
                        void* workspace, size_t workspace_bytes, FrontArgs* f, PagedPlan* plan,
                        uint64_t** keys, const void** dummy) {
  STK_REQUIRE(check_paged(dtype, requests, hq, hkv, nb, b, d, pages, topk, sp));
  STK_REQUIRE(q && k_pages && v_pages && lo_pages && hi_pages && table && nblocks,
              "null pointer");
  STK_REQUIRE(sp == 0 || (predicted && m && l && u), "null pointer");
  STK_REQUIRE(stk_bounds_ok(dtype, bounds_dtype),
              "lo and hi pages must be FP32 or the pages' 16-bit type");
  STK_REQUIRE(workspace && workspace_bytes >= stk_paged_workspace_bytes(requests, hq, nb),
              "workspace too small");
  const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_pages) |
                          reinterpret_cast<uintptr_t>(v_pages) |
                          reinterpret_cast<uintptr_t>(lo_pages) |
                          reinterpret_cast<uintptr_t>(hi_pages) |
                          (sp ? reinterpret_cast<uintptr_t>(u) : 0);
  plan->hq = requests * hq;
  plan->hkv = requests * hkv;
  const char* why = plan_step(dtype, plan->hq, plan->hkv, nb, b, d, topk < nb ? topk : nb,
                              sp > 0 ? sp : 1, IT_I32, align, &plan->s);
  STK_REQUIRE(why == nullptr, why ? why : "");
  *keys = static_cast<uint64_t*>(workspace);
  *dummy = static_cast<char*>(workspace) +
           stk_align((size_t)requests * hq * nb * sizeof(uint64_t));
  *f = make_front_args(q, k_pages, v_pages, dtype, plan->hq, plan->hkv, nb, b, d, lo_pages,
                       hi_pages, bounds_dtype != 0, predicted, sp, m, l, u, *keys, plan->s);
  f->pg = Paging{table, nblocks, hkv, pages, ntokens, nullptr, 0};
  return STK_OK;
}

STK_API int stk_paged_step(const void* q, const void* k_pages, const void* v_pages, int dtype,
                           int requests, int hq, int hkv, int nb, int b, int d, int pages,
                           const void* lo_pages, const void* hi_pages, int bounds_dtype,
                           const int32_t* block_table, const int32_t* nblocks,
                           const int32_t* ntokens, int topk, const int32_t* predicted, int sp,
                           int union_mode, int32_t* selected, float* m, float* l, float* u,
                           float* out, void* workspace, size_t workspace_bytes, void* stream) {
  FrontArgs f{};
  PagedPlan plan{};
  uint64_t* keys = nullptr;
  const void* dummy = nullptr;
  int rc = paged_common(q, k_pages, v_pages, dtype, requests, hq, hkv, nb, b, d, pages, lo_pages,
                        hi_pages, bounds_dtype, block_table, nblocks, ntokens, topk, predicted,
                        sp, m, l, u, workspace, workspace_bytes, &f, &plan, &keys, &dummy);
  if (rc) return rc;
  STK_REQUIRE(selected && out, "null pointer");
  TailArgs t{};
  t.kv = KV{q, k_pages, v_pages, plan.hq, plan.hkv, nb, b, d};
  t.keys = keys; t.k = topk; t.ids = selected;
  // with no predicted rows the tail's always-issued loads of slot 0 read the
  // dummy (their values are discarded)
  t.p = sp ? predicted : static_cast<const int32_t*>(dummy); t.sp = sp;
  t.pm = sp ? m : static_cast<const float*>(dummy);
  t.pl = sp ? l : static_cast<const float*>(dummy);
  t.pu = sp ? u : static_cast<const float*>(dummy);
  t.uni = union_mode ? 1 : 0; t.out = out;
  t.pg = f.pg;
  hipStream_t st = (hipStream_t)stream;
  rc = launch_front_pg(dtype, f, plan.s, st);
  if (rc) return rc;
  return launch_tail_pg(dtype, t, plan.s, st);
}

STK_API int stk_paged_signed_step(const void* q, const void* k_pages, const void* v_pages,
                                  int dtype, int requests, int hq, int hkv, int nb, int b, int d,
                                  int pages, const void* lo_pages, const void* hi_pages,
                                  int bounds_dtype, const int32_t* block_table,
                                  const int32_t* nblocks,
                                  const int32_t* ntokens, int topk, const int32_t* predicted,
                                  int sp, int hybrid, float mass_threshold, float min_remaining,
                                  float cancellation_tol, float max_extra_mass,
                                  int32_t* selected, float* m, float* l, float* u, float* out,
                                  uint8_t* fallback, float* remaining, uint8_t* approx,
                                  float* extra, int32_t* positive, int32_t* total,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  FrontArgs f{};
  PagedPlan plan{};
  uint64_t* keys = nullptr;
  const void* dummy = nullptr;
  int rc = paged_common(q, k_pages, v_pages, dtype, requests, hq, hkv, nb, b, d, pages, lo_pages,
                        hi_pages, bounds_dtype, block_table, nblocks, ntokens, topk, predicted,
                        sp, m, l, u, workspace, workspace_bytes, &f, &plan, &keys, &dummy);
  if (rc) return rc;
  STK_REQUIRE(selected && out && fallback && remaining && positive && total, "null pointer");
  STK_REQUIRE(!(max_extra_mass > 0.f) || (approx && extra),
              "max_extra_mass > 0 needs the approx and extra outputs");
  STK_REQUIRE(max_extra_mass >= 0.f && max_extra_mass <= 1.f, "max_extra_mass must be in [0,1]");
  STK_REQUIRE(mass_threshold >= 0.f && mass_threshold <= 1.f,
              "mass_threshold must be in [0,1]");
  STailArgs t{};
  t.kv = KV{q, k_pages, v_pages, plan.hq, plan.hkv, nb, b, d};
  t.keys = keys; t.k = topk; t.ids = selected;
  t.p = sp ? predicted : static_cast<const int32_t*>(dummy); t.sp = sp;
  t.pm = sp ? m : static_cast<const float*>(dummy);
  t.pl = sp ? l : static_cast<const float*>(dummy);
  t.pu = sp ? u : static_cast<const float*>(dummy);
  t.hybrid = hybrid ? 1 : 0;
  t.tau = mass_threshold; t.min_remaining = min_remaining; t.cancel_tol = cancellation_tol;
  t.eps = max_extra_mass;
  t.out = out; t.bad = fallback; t.remain = remaining;
  t.approx = max_extra_mass > 0.f ? approx : nullptr;
  t.extra = max_extra_mass > 0.f ? extra : nullptr;
  t.pos = positive; t.total = total;
  t.pg = f.pg;
  hipStream_t st = (hipStream_t)stream;
  rc = launch_front_pg(dtype, f, plan.s, st);
  if (rc) return rc;
  return launch_stail_pg(dtype, t, plan.s, st);
}

}  // extern "C"
