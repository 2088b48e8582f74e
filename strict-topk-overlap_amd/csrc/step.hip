// The speculative decode step on one stream: one launch (k_step1, step1.hpp)
// where it covers the shape, otherwise two.
//
// The reference runs select and speculate on two streams and joins them
// before the repair (benchmarks/run_benchmark.py:99-118, overlap_run).  On
// MI355X the two branches of a captured fork/join do not run concurrently,
// so the overlap is scheduled inside a grid.  The two-launch form is:
//   k_front        one grid whose workgroups are either scoring workgroups
//                  (bound score of a chunk of blocks -> 64-bit keys) or
//                  speculation workgroups (per-block softmax states of the
//                  predicted blocks, one wave per (query head, slot)), the two
//                  roles interleaved evenly inside every XCD so both
//                  streams of HBM traffic run side by side on all of them;
//   k_tail         one workgroup per query head: exact top-K of the head's
//                  keys (written out as the selected IDs, ascending), then the
//                  saved / union repair, laid out around two dependent memory
//                  round trips (everything known up front, then the missed
//                  blocks' tiles).
// The arithmetic is that of stk_select_blocks, stk_block_partials and
// stk_gqa_repair; results are identical up to FP32 reduction order.
#include <atomic>
#include <mutex>

#include "step1.hpp"
#include "step_small.hpp"

namespace stk {

const char* plan_step(int dtype, int hq, int hkv, int n, int b, int d, int topk, int sp,
                      int pred_dtype, uintptr_t align, StepShape* s) {
  if (dtype != DT_BF16 && dtype != DT_F16) return "the fused step takes bf16 or fp16 Q/K/V";
  if (pred_dtype != IT_I32) return "the fused step takes int32 predicted IDs";
  s->nch = tok_nch(dtype, d, b, align);
  if (!s->nch)
    return "the fused step needs D in {64, 128, 256}, B a multiple of 16 and 16-byte aligned Q/K/V";
  if (n > 8192) return "the fused step supports at most 8192 blocks";
  if (topk < 1 || topk > n || sp < 1) return "bad topk or predicted width";
  const int G = hq / hkv;
  s->passes = d / 64;
  s->steps = s->passes <= 2 ? 2 : 1;
  s->gt = G == 1 ? 1 : (G == 2 ? 2 : (s->passes <= 2 ? 4 : 2));
  if (s->passes > 2 && s->gt > 2) s->gt = 2;
  s->kpt = n <= kTailThreads * 4 ? 4 : (n <= kTailThreads * 8 ? 8 : 16);
  s->up = tok_up(b);
  s->one = b == 16 * s->up;
  if (topk > kTailMaxK || sp > kTailMaxK) return "the fused step takes at most 256 selected and predicted IDs";
  // predicted states held by the tail: sp rows over 2048 / D rows per pass
  const int per_pass = kTailThreads * 4 / d;
  const int rows = (sp + per_pass - 1) / per_pass;
  if (rows > 16) return "the fused step needs SP * D <= 32768";
  s->rpt = rows <= 4 ? 4 : 16;
  return nullptr;
}

FrontArgs make_front_args(const void* q, const void* k, const void* v, int dtype, int hq,
                          int hkv, int n, int b, int d, const void* lo, const void* hi, int lb,
                          const void* predicted, int sp, float* m, float* l, float* u,
                          uint64_t* keys, const StepShape& s) {
  FrontArgs f{};
  f.sc.q = q; f.sc.qtype = dtype; f.sc.lo = lo; f.sc.hi = hi; f.sc.lb = lb;
  f.sc.hq = hq; f.sc.hkv = hkv; f.sc.n = n; f.sc.d = d;
  f.sc.scores = nullptr; f.sc.keys = keys;
  f.sc.chunks = (n + kScoreWaves * 4 * s.steps - 1) / (kScoreWaves * 4 * s.steps);
  f.st.q = q; f.st.k = k; f.st.v = v; f.st.ids = predicted; f.st.itype = IT_I32;
  f.st.hq = hq; f.st.hkv = hkv; f.st.n = n; f.st.b = b; f.st.d = d; f.st.s = sp;
  f.st.m = m; f.st.l = l; f.st.u = u;
  f.score_wgs = hkv * f.sc.chunks;
  f.total_wgs = f.score_wgs + (int)(((int64_t)hq * sp + 3) / 4);
  return f;
}

}  // namespace stk

using namespace stk;

// ---- flag slots of the one-launch step
//
// k_step1's roles hand over through flags that must be zero before a launch
// and that every launch leaves zero.  They live in `g_step1_ctl`, static
// device memory (zero when the library is loaded), in kCtlSlots slots of
// kCtlSlotWords words: each stream that runs the step takes a slot of its own
// on first use, so launches in flight on different streams never share flags,
// and launches on one stream are ordered.  The last word of a slot counts
// timed-out waits.  With every slot taken (or a shape whose flags exceed a
// slot) the step runs as two launches.  In host code `g_step1_ctl` names a
// host-side stand-in: its device address comes from hipGetSymbolAddress.
static constexpr int kCtlSlots = 64;
static constexpr size_t kCtlSlotWords = 16384;
static __device__ __align__(256) uint32_t g_step1_ctl[kCtlSlots * kCtlSlotWords];

static constexpr int kMaxDevices = 64;
static std::mutex g_ctl_mu;
// The one launch's longest wait and, for failure tests only, whether its
// producers skip their flags (stk_step1_test_hook).
static std::atomic<uint64_t> g_step1_spin{kSpinTicks};
static std::atomic<int> g_step1_drop{0};
static struct {
  uint32_t* base;
  hipStream_t streams[kCtlSlots];
  int used;
} g_ctl_tab[kMaxDevices];

// True when `stream` is being captured into a graph.
static bool capturing(hipStream_t stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

// The slot of `stream` (nullptr when none is free or `words` exceed a slot).
static int ctl_slot(hipStream_t stream, size_t words, uint32_t** out) {
  *out = nullptr;
  if (words > kCtlSlotWords - 1) return STK_OK;
  hipDevice_t dev = 0;
  hipError_t e = hipStreamGetDevice(stream, &dev);
  if (e != hipSuccess) {
    stk_set_error("hipStreamGetDevice failed: %s", hipGetErrorString(e));
    return STK_EHIP;
  }
  if (dev < 0 || dev >= kMaxDevices) return STK_OK;
  std::lock_guard<std::mutex> guard(g_ctl_mu);
  auto& tab = g_ctl_tab[dev];
  if (!tab.base) {
    if (capturing(stream)) {
      stk_set_error("the step's device memory is looked up on a device's first call, which "
                    "must not be under stream capture: call stk_step_prepare() first");
      return STK_EINVAL;
    }
    int cur = 0;
    e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_step1_ctl));
    const hipError_t restore = cur != dev ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess || restore != hipSuccess || !p) {
      stk_set_error("flag slots on device %d: %s", (int)dev,
                    hipGetErrorString(e != hipSuccess ? e : restore));
      return STK_EHIP;
    }
    tab.base = static_cast<uint32_t*>(p);
  }
  int slot = -1;
  for (int i = 0; i < tab.used; ++i)
    if (tab.streams[i] == stream) slot = i;
  if (slot < 0 && tab.used < kCtlSlots) {
    slot = tab.used++;
    tab.streams[slot] = stream;
  }
  if (slot >= 0) *out = tab.base + (size_t)slot * kCtlSlotWords;
  return STK_OK;
}

int stk::launch_front(int dtype, const FrontArgs& f, const StepShape& s, hipStream_t st) {
  return launch::front<false>(dtype, f, s, st);
}

extern "C" {

STK_API size_t stk_step_workspace_bytes(int hq, int hkv, int n, int d, int topk) {
  (void)hkv; (void)d; (void)topk;
  if (hq <= 0 || n <= 0) return 0;
  return stk_align((size_t)hq * n * sizeof(uint64_t));
}

STK_API int stk_step_supported(int dtype, int hq, int hkv, int n, int b, int d, int topk, int sp,
                               int pred_dtype) {
  StepShape s{};
  if (hq <= 0 || hkv <= 0 || hq % hkv) return 0;
  return plan_step(dtype, hq, hkv, n, b, d, topk, sp, pred_dtype, 0, &s) == nullptr;
}

static int step_call(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                     int n, int b, int d, const void* lo, const void* hi, int bounds_dtype,
                     int topk,
                     const void* predicted, int pred_dtype, int sp, int union_mode,
                     int32_t* selected, float* m, float* l, float* u, float* out,
                     void* workspace, size_t workspace_bytes, void* stream, bool front,
                     bool tail) {
  STK_REQUIRE(stk_check_kv(dtype, hq, hkv, n, b, d));
  STK_REQUIRE(q && k && v && predicted && m && l && u, "null pointer");
  STK_REQUIRE(!front || (lo && hi), "null pointer");
  STK_REQUIRE(!front || stk_bounds_ok(dtype, bounds_dtype),
              "lo and hi must be FP32 or the element type of Q/K/V");
  STK_REQUIRE(!tail || (selected && out), "null pointer");
  STK_REQUIRE(workspace && workspace_bytes >= stk_step_workspace_bytes(hq, hkv, n, d, topk),
              "workspace too small");
  const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(u) |
                          (front ? reinterpret_cast<uintptr_t>(lo) | reinterpret_cast<uintptr_t>(hi)
                                 : 0);
  StepShape s{};
  const char* why = plan_step(dtype, hq, hkv, n, b, d, topk, sp, pred_dtype, align, &s);
  STK_REQUIRE(why == nullptr, why ? why : "");
  uint64_t* keys = static_cast<uint64_t*>(workspace);
  const FrontArgs f = make_front_args(q, k, v, dtype, hq, hkv, n, b, d, lo, hi,
                                      bounds_dtype != 0, predicted, sp, m, l, u, keys, s);
  TailArgs t{};
  t.kv = KV{q, k, v, hq, hkv, n, b, d};
  t.keys = keys; t.k = topk; t.ids = selected;
  t.p = static_cast<const int32_t*>(predicted); t.sp = sp;
  t.pm = m; t.pl = l; t.pu = u; t.uni = union_mode ? 1 : 0; t.out = out;
  hipStream_t st = (hipStream_t)stream;
  if (front && tail && small_covers(dtype, hq, hkv, n, b, d, topk, sp, bounds_dtype, align)) {
    // small shapes: one workgroup per query head, no hand-off
    SmallArgs sa{q, k, v, lo, hi, hq, hkv, n, d, t.p, sp, topk, t.uni, selected, m, l, u, out};
    return launch_small(dtype, sa, bounds_dtype, st);
  }
  if (front && tail && step1_covers(dtype, hq, hkv, b, d, s)) {
    // one launch, its flags in this stream's slot (none free: two launches)
    uint32_t* ctl = nullptr;
    const int rc = ctl_slot(st, step1_ctl_words(hq, n, sp), &ctl);
    if (rc) return rc;
    if (ctl)
      return launch_step1(dtype, f, t, s, ctl, kCtlSlotWords - 1, ctl + kCtlSlotWords - 1,
                          g_step1_spin.load(), g_step1_drop.load(), st);
  }
  if (front) {
    const int rc = launch_front(dtype, f, s, st);
    if (rc) return rc;
  }
  if (!tail) return STK_OK;
  return launch_tail(dtype, t, s, st);
}

STK_API int stk_speculative_step(const void* q, const void* k, const void* v, int dtype, int hq,
                                 int hkv, int n, int b, int d, const void* lo, const void* hi,
                                 int bounds_dtype, int topk, const void* predicted, int pred_dtype, int sp,
                                 int union_mode, int32_t* selected, float* m, float* l, float* u,
                                 float* out, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  return step_call(q, k, v, dtype, hq, hkv, n, b, d, lo, hi, bounds_dtype, topk, predicted,
                   pred_dtype, sp, union_mode, selected, m, l, u, out, workspace,
                   workspace_bytes, stream, true, true);
}

STK_API int stk_step1_supported(int dtype, int hq, int hkv, int n, int b, int d, int topk,
                                int sp, int pred_dtype) {
  StepShape s{};
  if (hq <= 0 || hkv <= 0 || hq % hkv) return 0;
  if (plan_step(dtype, hq, hkv, n, b, d, topk, sp, pred_dtype, 0, &s)) return 0;
  return step1_covers(dtype, hq, hkv, b, d, s) &&
         step1_ctl_words(hq, n, sp) < kCtlSlotWords ? 1 : 0;   // the last word counts time-outs
}

STK_API int stk_step_small_supported(int dtype, int hq, int hkv, int n, int b, int d, int topk,
                                     int sp, int pred_dtype, int bounds_dtype) {
  StepShape s{};
  if (hq <= 0 || hkv <= 0 || hq % hkv) return 0;
  if (plan_step(dtype, hq, hkv, n, b, d, topk, sp, pred_dtype, 0, &s)) return 0;
  return small_covers(dtype, hq, hkv, n, b, d, topk, sp, bounds_dtype, 0) ? 1 : 0;
}

STK_API int stk_step1_timeouts(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  int count = 0;
  for (int i = 0; i < kCtlSlots; ++i) {
    uint32_t v = 0;
    if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_step1_ctl), sizeof(v),
                            ((size_t)i * kCtlSlotWords + kCtlSlotWords - 1) * sizeof(uint32_t),
                            hipMemcpyDeviceToHost) != hipSuccess)
      return -1;
    count += v != 0;
  }
  return count;
}

STK_API int stk_step1_test_hook(unsigned long long spin_ticks, int drop_flags) {
  g_step1_spin.store(spin_ticks);
  g_step1_drop.store(drop_flags ? 1 : 0);
  const uint32_t zero = 0;
  for (int i = 0; i < kCtlSlots; ++i) {
    const hipError_t e = hipMemcpyToSymbol(
        HIP_SYMBOL(g_step1_ctl), &zero, sizeof(zero),
        ((size_t)i * kCtlSlotWords + kCtlSlotWords - 1) * sizeof(uint32_t), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      stk_set_error("clearing the time-out counters: %s", hipGetErrorString(e));
      return STK_EHIP;
    }
  }
  return STK_OK;
}

// ---- the allocation-free variant of stk_speculative_step
//
// Its score keys live in `scratch`, one array per GPU, sized for
// hq * n <= kNoAllocMaxKeys (4 MiB).  In host code `scratch` names a host-side
// stand-in, never the device copy: the device address comes from
// hipGetSymbolAddress, once per device with that device current, and only
// that address is passed to kernels.  Every call on one GPU shares the array
// and the last call's keys stay in it; the front writes every key the tail
// reads (keys [h, 0, n) of each head), so nothing needs clearing.  Calls that
// overlap on one GPU (two streams at once) race on it.
constexpr size_t kNoAllocMaxKeys = (size_t)1 << 19;
static __device__ __align__(256) uint64_t scratch[kNoAllocMaxKeys];

static std::mutex g_scratch_mu;
static void* g_scratch_dev[kMaxDevices];

// The device address of `scratch` on the device that runs `stream`.
static int scratch_address(hipStream_t stream, void** out) {
  hipDevice_t dev = 0;
  hipError_t e = hipStreamGetDevice(stream, &dev);
  if (e != hipSuccess) {
    stk_set_error("hipStreamGetDevice failed: %s", hipGetErrorString(e));
    return STK_EHIP;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    stk_set_error("device ordinal %d out of range", (int)dev);
    return STK_EINVAL;
  }
  std::lock_guard<std::mutex> guard(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    if (capturing(stream)) {
      stk_set_error("the allocation-free step's scratch is looked up on a device's first call, "
                    "which must not be under stream capture: call stk_step_prepare() first");
      return STK_EINVAL;
    }
    int cur = 0;
    e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t restore = cur != dev ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess || restore != hipSuccess || !p) {
      stk_set_error("scratch address on device %d: %s", (int)dev,
                    hipGetErrorString(e != hipSuccess ? e : restore));
      return STK_EHIP;
    }
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return STK_OK;
}

STK_API size_t stk_step_noalloc_max_keys(void) { return kNoAllocMaxKeys; }

STK_API int stk_step_prepare(void) {
  hipStream_t st = nullptr;   // the null stream of the current device: never capturing
  void* ws = nullptr;
  int rc = scratch_address(st, &ws);
  if (rc) return rc;
  uint32_t* ctl = nullptr;
  return ctl_slot(st, 0, &ctl);
}

STK_API int stk_speculative_step_noalloc(const void* q, const void* k, const void* v, int dtype,
                                         int hq, int hkv, int n, int b, int d, const void* lo,
                                         const void* hi, int bounds_dtype, int topk,
                                         const void* predicted,
                                         int pred_dtype, int sp, int union_mode,
                                         int32_t* selected, float* m, float* l, float* u,
                                         float* out, void* stream) {
  STK_REQUIRE(stk_check_kv(dtype, hq, hkv, n, b, d));
  STK_REQUIRE(q && k && v && lo && hi && predicted && selected && m && l && u && out,
              "null pointer");
  STK_REQUIRE((size_t)hq * (size_t)n <= kNoAllocMaxKeys,
              "the allocation-free step holds at most 524288 score keys (Hq * N)");
  void* ws = nullptr;
  const int rc = scratch_address((hipStream_t)stream, &ws);
  if (rc) return rc;
  return step_call(q, k, v, dtype, hq, hkv, n, b, d, lo, hi, bounds_dtype, topk, predicted,
                   pred_dtype, sp, union_mode, selected, m, l, u, out, ws,
                   kNoAllocMaxKeys * sizeof(uint64_t), stream, true, true);
}

STK_API int stk_step_front(const void* q, const void* k, const void* v, int dtype, int hq,
                           int hkv, int n, int b, int d, const void* lo, const void* hi,
                           int bounds_dtype, int topk, const void* predicted, int pred_dtype, int sp, float* m,
                           float* l, float* u, void* workspace, size_t workspace_bytes,
                           void* stream) {
  return step_call(q, k, v, dtype, hq, hkv, n, b, d, lo, hi, bounds_dtype, topk, predicted,
                   pred_dtype, sp, 0, nullptr, m, l, u, nullptr, workspace, workspace_bytes,
                   stream, true, false);
}

STK_API int stk_step_tail(const void* q, const void* k, const void* v, int dtype, int hq,
                          int hkv, int n, int b, int d, int topk, const void* predicted,
                          int pred_dtype, int sp, int union_mode, const float* m, const float* l,
                          const float* u, int32_t* selected, float* out, void* workspace,
                          size_t workspace_bytes, void* stream) {
  return step_call(q, k, v, dtype, hq, hkv, n, b, d, nullptr, nullptr, 0, topk, predicted,
                   pred_dtype, sp, union_mode, selected, const_cast<float*>(m),
                   const_cast<float*>(l), const_cast<float*>(u), out, workspace,
                   workspace_bytes, stream, false, true);
}

}  // extern "C"
