// Min/max query-sign bound scorer plus exact top-K selection.
//
// Reference: strict_topk/selector.py:8-20,23-43 (_score, block_scores,
// select_blocks) and strict_topk/gqa.py:15-26,145-161 (_bound_score,
// select_blocks), which end in torch.topk(sorted=False).
//
// Score contract: score[h,n] = sum_d q_d * (q_d >= 0 ? hi : lo)[h/G, n, d]
// in FP64.  Products of a 16/32-bit q and an FP32 bound are exact in FP64;
// 16 lanes share a block, lane c summing dims 64*j + 4*c + t (j ascending,
// t = 0..3) from +0.0, then the lanes combine with an xor butterfly
// (8, 4, 2, 1).  Selection contract: the K largest (score, -index) pairs,
// so ties go to the lower block index; IDs are written in ascending block
// order.  NaN scores rank below -inf.
//
// Launch structure (MI355X):
//   k_score  -- HBM-bound scan of lo/hi.  One workgroup = 4 waves covers
//               16 * STEPS consecutive blocks of one KV head for all G query
//               heads of that head (lo/hi read once per KV head); every lane
//               issues all its 16-byte loads before any arithmetic.  Writes
//               an order-preserving 64-bit key per (query head, block).
//   k_topk   -- one 256-thread workgroup per query head: the value-bin
//               selection of topk_bins.hpp over the row's keys held in
//               registers (radix select as its fallback), then a block-wide
//               scan writes the selected IDs in index order.
#include "score.hpp"
#include "topk_bins.hpp"
#include "api.hpp"

namespace stk {

constexpr int kTopkThreads = 256;
constexpr int kTopkWide = 1024;     // threads of k_topk_wide (16 waves)
constexpr int kWideRows = 4;        // rows up to which k_topk_wide is used
constexpr int kFewRows = 256;       // rows up to which a row gets four keys per thread
template <typename Q, int P, int STEPS, bool FULL, int GT>
__global__ __launch_bounds__(256) void k_score(ScoreArgs a) {
  score_wg<Q, P, STEPS, FULL, GT>(a, blockIdx.x);
}

struct TopkArgs {
  const uint64_t* keys;
  int n, k;
  int32_t* ids;
};

// One row's selection by value bins (topk_bins.hpp): KPT keys per thread,
// the selected indices ranked by one scan and written in ascending order.
template <int KPT>
__device__ __forceinline__ void topk_row(const TopkArgs& a, TopkBinsLds& tb, int* s_scan) {
  const uint64_t* rk = a.keys + (size_t)blockIdx.x * a.n;
  int32_t* out = a.ids + (size_t)blockIdx.x * a.k;
  uint64_t key[KPT];
  topk_load<KPT>(rk, a.n, key);
  const uint32_t flags = topk_bins_flags<KPT>(key, a.n, a.k, tb, [] {});
  int total;
  int pos = block_excl_scan1(__popc(flags), s_scan, &total);
#pragma unroll
  for (int i = 0; i < KPT; ++i)
    if ((flags >> i) & 1u) out[pos++] = threadIdx.x * KPT + i;
}

// One workgroup per row (TopkArgs.keys[row, 0..n)).
template <int KPT>
__global__ __launch_bounds__(kTopkThreads) void k_topk(TopkArgs a) {
  __shared__ TopkBinsLds tb;
  __shared__ int s_scan[kTopkThreads / STK_WAVE];
  topk_row<KPT>(a, tb, s_scan);
}

// The same selection with 1024 threads (KPT keys each), for shapes with few
// rows, where one workgroup per row leaves most of the chip idle and a
// row's phases are the latency.
template <int KPT>
__global__ __launch_bounds__(kTopkWide) void k_topk_wide(TopkArgs a) {
  __shared__ TopkBinsLds tb;
  __shared__ int s_scan[kTopkWide / STK_WAVE];
  topk_row<KPT>(a, tb, s_scan);
}

// Rows longer than 8192 keys: the same selection with keys re-read from
// global memory in every pass (thread t owns a contiguous index range).
__global__ __launch_bounds__(kTopkThreads) void k_topk_long(TopkArgs a) {
  __shared__ int hist[256];
  __shared__ int tmp[kTopkThreads / STK_WAVE];
  __shared__ uint64_t red64[2][kTopkThreads / STK_WAVE];
  __shared__ int pick[2];
  const int row = blockIdx.x;
  const uint64_t* rk = a.keys + (size_t)row * a.n;
  const int per = (a.n + kTopkThreads - 1) / kTopkThreads;
  const int b0 = threadIdx.x * per;
  const int b1 = min(a.n, b0 + per);
  uint64_t vor = 0ull, vand = ~0ull;
  for (int i = b0; i < b1; ++i) {
    vor |= rk[i];
    vand &= rk[i];
  }
  vor = wave_or64(vor);
  vand = wave_and64(vand);
  if (lane_id() == 0) {
    red64[0][wave_id()] = vor;
    red64[1][wave_id()] = vand;
  }
  __syncthreads();
  vor = 0ull;
  vand = ~0ull;
  for (int w = 0; w < kTopkThreads / STK_WAVE; ++w) {
    vor |= red64[0][w];
    vand &= red64[1][w];
  }
  const uint64_t diff = vor ^ vand;
  uint64_t mask = ~0ull, prefix = vand;
  int need = a.k;
  if (diff != 0ull) {
    int start = 63 - __clzll((long long)diff);
    mask = start == 63 ? 0ull : ~0ull << (start + 1);
    prefix = vand & mask;
    while (true) {
      const int shift = start >= 7 ? start - 7 : 0;
      const int width = start - shift + 1;
      const uint64_t dmask = ((1ull << width) - 1ull);
      for (int i = threadIdx.x; i < 256; i += blockDim.x) hist[i] = 0;
      __syncthreads();
      for (int i = b0; i < b1; ++i) {
        uint64_t kk = rk[i];
        if ((kk & mask) == prefix) atomicAdd(&hist[(kk >> shift) & dmask], 1);
      }
      __syncthreads();
      if (wave_id() == 0) {
        int c[4], s = 0;
        for (int t = 0; t < 4; ++t) {
          c[t] = hist[255 - 4 * lane_id() - t];
          s += c[t];
        }
        int inc = wave_incl_scan(s);
        int above = inc - s;
        for (int t = 0; t < 4; ++t) {
          if (above < need && above + c[t] >= need) {
            pick[0] = 255 - 4 * lane_id() - t;
            pick[1] = above;
          }
          above += c[t];
        }
      }
      __syncthreads();
      const int bin = pick[0];
      const int above = pick[1];
      const int cnt = hist[bin];
      need -= above;
      prefix |= (uint64_t)bin << shift;
      mask |= dmask << shift;
      __syncthreads();
      if (cnt == need || shift == 0) break;
      start = shift - 1;
    }
  }
  int eq = 0;
  for (int i = b0; i < b1; ++i) eq += (rk[i] & mask) == prefix;
  int total;
  int eq_before = block_excl_scan(eq, tmp, &total);
  int cnt = 0;
  for (int i = b0; i < b1; ++i) {
    uint64_t km = rk[i] & mask;
    bool e = km == prefix;
    cnt += km > prefix || (e && eq_before < need);
    eq_before += e;
  }
  eq_before = block_excl_scan(eq, tmp, &total);
  int pos = block_excl_scan(cnt, tmp, &total);
  int32_t* out = a.ids + (size_t)row * a.k;
  for (int i = b0; i < b1; ++i) {
    uint64_t km = rk[i] & mask;
    bool e = km == prefix;
    if (km > prefix || (e && eq_before < need)) out[pos++] = i;
    eq_before += e;
  }
}

}  // namespace stk

using namespace stk;

static StkCheck check_select(int q_dtype, int hq, int hkv, int n, int d) {
  if (q_dtype < DT_F32 || q_dtype > DT_BF16) return {false, "unsupported q dtype"};
  if (hq <= 0 || hkv <= 0 || n <= 0 || d <= 0) return {false, "expected nonempty shapes"};
  if (hq % hkv) return {false, "Hq must be divisible by Hkv"};
  if (d > 1024) return {false, "head dimension above 1024 is not supported"};
  return {true, ""};
}

// Launch the scorer: blocks per workgroup = 4 waves * 4 blocks * STEPS.
template <typename Q>
static void launch_score_q(ScoreArgs& a, hipStream_t st) {
  const int passes = (a.d + 63) / 64;
  const bool full = a.d % 64 == 0 && (reinterpret_cast<uintptr_t>(a.lo) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(a.hi) & 15) == 0;
#define STK_SCORE(PP, SS, GG)                                                                  \
  do {                                                                                         \
    a.chunks = (a.n + kScoreWaves * 4 * SS - 1) / (kScoreWaves * 4 * SS);                       \
    if (full)                                                                                  \
      hipLaunchKernelGGL((k_score<Q, PP, SS, true, GG>), dim3(a.hkv * a.chunks), dim3(256), 0, st, a); \
    else                                                                                       \
      hipLaunchKernelGGL((k_score<Q, PP, SS, false, GG>), dim3(a.hkv * a.chunks), dim3(256), 0, st, a); \
  } while (0)
  const int G = a.hq / a.hkv;
  if (passes <= 1) {
    if (G <= 1) STK_SCORE(1, 2, 1);
    else if (G <= 2) STK_SCORE(1, 2, 2);
    else STK_SCORE(1, 2, 4);
  } else if (passes <= 2) {
    if (G <= 1) STK_SCORE(2, 2, 1);
    else if (G <= 2) STK_SCORE(2, 2, 2);
    else STK_SCORE(2, 2, 4);
  } else if (passes <= 4) {
    STK_SCORE(4, 1, 2);
  } else if (passes <= 8) {
    STK_SCORE(8, 1, 1);
  } else {
    STK_SCORE(16, 1, 1);
  }
#undef STK_SCORE
}

int stk_launch_score(const void* q, int q_dtype, const void* lo, const void* hi, int lb, int hq,
                     int hkv, int n, int d, float* scores, uint64_t* keys, hipStream_t st) {
  ScoreArgs a{};
  a.q = q; a.qtype = q_dtype; a.lo = lo; a.hi = hi; a.lb = lb;
  a.hq = hq; a.hkv = hkv; a.n = n; a.d = d;
  a.scores = scores; a.keys = keys;
  if (q_dtype == DT_BF16) launch_score_q<bf16s>(a, st);
  else if (q_dtype == DT_F16) launch_score_q<f16s>(a, st);
  else launch_score_q<float>(a, st);
  return stk_check_launch("k_score");
}

// 1024-thread rows for a few long rows (the shared selection's single row).
static bool wide_topk(int rows, int n) { return rows <= kWideRows && n > 1024 && n <= 16384; }

int stk_launch_topk(const uint64_t* keys, int rows, int n, int k, int32_t* ids, hipStream_t st) {
  TopkArgs t{keys, n, k, ids};
  const dim3 grid(rows), block(kTopkThreads);
  if (wide_topk(rows, n)) {
    const dim3 wb(kTopkWide);
    if (n <= 2048) hipLaunchKernelGGL(k_topk_wide<2>, grid, wb, 0, st, t);
    else if (n <= 4096) hipLaunchKernelGGL(k_topk_wide<4>, grid, wb, 0, st, t);
    else if (n <= 8192) hipLaunchKernelGGL(k_topk_wide<8>, grid, wb, 0, st, t);
    else hipLaunchKernelGGL(k_topk_wide<16>, grid, wb, 0, st, t);
    return stk_check_launch("k_topk_wide");
  }
  // up to 256 rows of 1024 < n <= 8192 keys: four keys per thread up to 4096
  // keys (512 or 1024 threads), eight above.  Measured on MI355X against 256
  // threads (select_blocks, IDs identical): 32 rows of 2048 keys 9.3 -> 8.5 us,
  // of 4000 keys 14.0 -> 11.7 us, of 8000 keys 25.8 -> 21.3 us; 128 rows of
  // 4000 keys 25.5 -> 22.9 us.  Rows past 256 keep the 256-thread kernels.
  if (rows <= kFewRows && n > 1024 && n <= 8192) {
    if (n <= 2048) hipLaunchKernelGGL(k_topk_wide<4>, grid, dim3(512), 0, st, t);
    else if (n <= 4096) hipLaunchKernelGGL(k_topk_wide<4>, grid, dim3(kTopkWide), 0, st, t);
    else hipLaunchKernelGGL(k_topk_wide<8>, grid, dim3(kTopkWide), 0, st, t);
    return stk_check_launch("k_topk_wide");
  }
  if (n <= 256) hipLaunchKernelGGL(k_topk<1>, grid, block, 0, st, t);
  else if (n <= 512) hipLaunchKernelGGL(k_topk<2>, grid, block, 0, st, t);
  else if (n <= 1024) hipLaunchKernelGGL(k_topk<4>, grid, block, 0, st, t);
  else if (n <= 2048) hipLaunchKernelGGL(k_topk<8>, grid, block, 0, st, t);
  else if (n <= 4096) hipLaunchKernelGGL(k_topk<16>, grid, block, 0, st, t);
  else if (n <= 8192) hipLaunchKernelGGL(k_topk<32>, grid, block, 0, st, t);
  else hipLaunchKernelGGL(k_topk_long, grid, block, 0, st, t);
  return stk_check_launch("k_topk");
}

extern "C" {

STK_API int stk_block_scores(const void* q, int q_dtype, const void* lo, const void* hi,
                             int bounds_dtype, int hq, int hkv, int n, int d, float* scores,
                             void* stream) {
  STK_REQUIRE(check_select(q_dtype, hq, hkv, n, d));
  STK_REQUIRE(q && lo && hi && scores, "null pointer");
  STK_REQUIRE(stk_bounds_ok(q_dtype, bounds_dtype),
              "lo and hi must be FP32 or the query's 16-bit type");
  return stk_launch_score(q, q_dtype, lo, hi, bounds_dtype != 0, hq, hkv, n, d, scores, nullptr,
                          (hipStream_t)stream);
}

STK_API size_t stk_select_workspace_bytes(int hq, int hkv, int n, int d, int topk) {
  if (hq <= 0 || hkv <= 0 || n <= 0 || d <= 0 || topk <= 0) return 0;
  return stk_align((size_t)hq * n * sizeof(uint64_t));
}

STK_API int stk_select_blocks(const void* q, int q_dtype, const void* lo, const void* hi,
                              int bounds_dtype, int hq, int hkv, int n, int d, int topk,
                              float* scores, int32_t* ids, void* workspace,
                              size_t workspace_bytes, void* stream) {
  STK_REQUIRE(check_select(q_dtype, hq, hkv, n, d));
  STK_REQUIRE(q && lo && hi && ids, "null pointer");
  STK_REQUIRE(stk_bounds_ok(q_dtype, bounds_dtype),
              "lo and hi must be FP32 or the query's 16-bit type");
  STK_REQUIRE(topk >= 1 && topk <= n, "selected index k out of range");
  STK_REQUIRE(workspace && workspace_bytes >= stk_select_workspace_bytes(hq, hkv, n, d, topk),
              "workspace too small");
  hipStream_t st = (hipStream_t)stream;
  uint64_t* keys = static_cast<uint64_t*>(workspace);
  int rc = stk_launch_score(q, q_dtype, lo, hi, bounds_dtype != 0, hq, hkv, n, d, scores, keys,
                            st);
  if (rc) return rc;
  return stk_launch_topk(keys, hq, n, topk, ids, st);
}

}  // extern "C"
