// Shared-selection indexer scorer: the QSA formula
//   score[n] = sum_h relu(iq_h . ik_n) / sqrt(D)
// over H indexer heads and N indexer keys (one per block), then one top-K
// shared by every query head.
//
// Reference: benchmarks/selector_window.py:126-142 (_indexer_scores,
// qsa_reference_scores) and :76-84 (the shared selector:
// scores.topk(topk, sorted=False), expanded to every query head).
//
// Score contract (so that IDs are bit-exact against the FP64 oracle): 16
// lanes per key; lane p sums dims [p*Q, p*Q + Q), Q = ceil(D / 16), in
// order, in FP64 (16-bit x 16-bit and FP32 x FP32 products are exact
// there); the 16 partials combine as a pairwise tree (the xor butterfly
// 1, 2, 4, 8: (s0 + s1) + (s2 + s3) and so on); relu (NaN kept, as
// torch.relu) per head; heads summed in order from 0.0; times
// inv = 1 / sqrt(D) (FP64, computed on the host: the reference's D**-.5
// factor).  The top-K is the selector's (ties toward the lower index, IDs
// ascending).
//
// k_indexer_v (16-bit keys, D = 128): each lane holds its 8 dims from one
// 16-byte load and its query slices in registers, so a key is one coalesced
// 256-byte row per 16 lanes and the four heads are four independent 8-FMA
// chains.  k_indexer serves every other shape with the same arithmetic.
#include <cmath>

#include "score.hpp"
#include "topk_bins.hpp"
#include "api.hpp"

namespace stk {

constexpr int kIdxMaxQ = 4096;   // H * D staged in LDS (FP64)

struct IndexerArgs {
  const void* iq; const void* ik;
  int h, n, d;
  double inv;          // 1 / sqrt(D)
  float* scores;       // may be null
  uint64_t* keys;
};

constexpr int kIdxLanes = 16;    // lanes per key

// Pairwise tree over the 16 lanes of a key (IEEE addition is commutative,
// so both lanes of every exchange hold the same sum).
__device__ __forceinline__ double key_tree(double x) {
  x += __shfl_xor(x, 1);
  x += __shfl_xor(x, 2);
  x += __shfl_xor(x, 4);
  x += __shfl_xor(x, 8);
  return x;
}

__device__ __forceinline__ double relu_nan(double x) { return (x > 0.0 || x != x) ? x : 0.0; }

template <typename T>
__global__ __launch_bounds__(256) void k_indexer(IndexerArgs a) {
  __shared__ double s_q[kIdxMaxQ];
  const T* iq = reinterpret_cast<const T*>(a.iq);
  for (int x = threadIdx.x; x < a.h * a.d; x += blockDim.x) s_q[x] = (double)cvt(iq[x]);
  __syncthreads();
  const int key = blockIdx.x * (blockDim.x / kIdxLanes) + threadIdx.x / kIdxLanes;
  const int p = threadIdx.x % kIdxLanes;
  const bool ok = key < a.n;
  const int qd = (a.d + kIdxLanes - 1) / kIdxLanes;
  const int d0 = p * qd < a.d ? p * qd : a.d;
  const int d1 = d0 + qd < a.d ? d0 + qd : a.d;
  const T* row = reinterpret_cast<const T*>(a.ik) + (size_t)(ok ? key : 0) * a.d;
  double sc = 0.0;
  for (int hh = 0; hh < a.h; ++hh) {
    const double* qh = s_q + hh * a.d;
    double acc = 0.0;
    for (int i = d0; i < d1; ++i) acc = fma((double)cvt(row[i]), qh[i], acc);
    sc += relu_nan(key_tree(acc));
  }
  sc = sc * a.inv;
  if (ok && p == 0) {
    if (a.scores) a.scores[key] = (float)sc;
    a.keys[key] = score_key(sc);
  }
}

// The score of `key` (lane p of its 16; every lane returns the sum).
template <typename T, int H>
__device__ __forceinline__ double indexer_score_v(const IndexerArgs& a, int key, int p, bool ok) {
  constexpr int D = 128;
  // this lane's 8 dims of the key row (one 16-byte load) and of every query
  const uint4 kr = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(a.ik) +
                                                   (size_t)(ok ? key : 0) * D + 8 * p);
  const T* iq = reinterpret_cast<const T*>(a.iq);
  uint4 qr[H];
#pragma unroll
  for (int hh = 0; hh < H; ++hh)
    qr[hh] = *reinterpret_cast<const uint4*>(iq + (size_t)hh * D + 8 * p);
  double kv[8];
  {
    const uint32_t w[4] = {kr.x, kr.y, kr.z, kr.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      kv[2 * e] = (double)cvt(T{uint16_t(w[e] & 0xffffu)});
      kv[2 * e + 1] = (double)cvt(T{uint16_t(w[e] >> 16)});
    }
  }
  double part[H];
#pragma unroll
  for (int hh = 0; hh < H; ++hh) {
    const uint32_t w[4] = {qr[hh].x, qr[hh].y, qr[hh].z, qr[hh].w};
    double acc = 0.0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc = fma(kv[2 * e], (double)cvt(T{uint16_t(w[e] & 0xffffu)}), acc);
      acc = fma(kv[2 * e + 1], (double)cvt(T{uint16_t(w[e] >> 16)}), acc);
    }
    part[hh] = acc;
  }
  double sc = 0.0;
#pragma unroll
  for (int hh = 0; hh < H; ++hh) sc += relu_nan(key_tree(part[hh]));
  return sc * a.inv;
}

template <typename T, int H>
__global__ __launch_bounds__(256) void k_indexer_v(IndexerArgs a) {
  const int key = blockIdx.x * (blockDim.x / kIdxLanes) + threadIdx.x / kIdxLanes;
  const int p = threadIdx.x % kIdxLanes;
  const bool ok = key < a.n;
  const double sc = indexer_score_v<T, H>(a, key, p, ok);
  if (ok && p == 0) {
    if (a.scores) a.scores[key] = (float)sc;
    a.keys[key] = score_key(sc);
  }
}

// ids[r, :] = ids[0, :] for r in [1, rows): x = column, rows from blockIdx.y
__global__ __launch_bounds__(256) void k_rows_copy(int32_t* ids, int rows, int k) {
  const int x = blockIdx.x * blockDim.x + threadIdx.x;
  if (x >= k) return;
  const int32_t v = ids[x];
  for (int r = blockIdx.y + 1; r < rows; r += gridDim.y) ids[(size_t)r * k + x] = v;
}

// ---- the shared top-K and its rows
//
// The selection is one row of n keys, the same for every query head, so the
// output is rows copies of topk IDs (393 KB at 48 rows of 2048).  T
// workgroups of 1024 threads each rank the whole row (value bins,
// topk_bins.hpp, KPT keys per thread), stage the ranked IDs in LDS and write
// rows j, j + T, ... (16 bytes per store where the rows allow it): the rows
// leave from T CUs at once, where one workgroup alone would take several
// microseconds to store them, and no copy kernel follows.
constexpr int kShThreads = 1024;
constexpr int kShMaxN = 16 * kShThreads;   // KPT <= 16
constexpr int kShMaxK = 8192;              // ranked IDs staged in LDS
constexpr int kShRowsPer = 4;              // output rows per workgroup
constexpr int kShMaxWgs = 64;              // past 256 rows a workgroup writes more than four

struct SharedTopkArgs {
  const uint64_t* keys;
  int n, k, rows;
  int32_t* ids;   // [rows, k]
  int vec;        // k % 4 == 0 and ids 16-byte aligned
};

template <int KPT>
__global__ __launch_bounds__(kShThreads) void k_topk_shared(SharedTopkArgs a) {
  __shared__ TopkBinsLds tb;
  __shared__ int s_scan[kShThreads / STK_WAVE];
  __shared__ __align__(16) int s_ids[kShMaxK];
  const int tid = threadIdx.x;
  uint64_t key[KPT];
  topk_load<KPT>(a.keys, a.n, key);
  const uint32_t flags = topk_bins_flags<KPT>(key, a.n, a.k, tb, [] {});
  int total;
  int pos = block_excl_scan1(__popc(flags), s_scan, &total);
#pragma unroll
  for (int i = 0; i < KPT; ++i)
    if ((flags >> i) & 1u) s_ids[pos++] = tid * KPT + i;
  __syncthreads();
  if (a.vec) {
    const int k4 = a.k / 4;
    const int4* src = reinterpret_cast<const int4*>(s_ids);
    for (int r = blockIdx.x; r < a.rows; r += gridDim.x) {
      int4* o = reinterpret_cast<int4*>(a.ids + (size_t)r * a.k);
      for (int x = tid; x < k4; x += kShThreads) o[x] = src[x];
    }
  } else {
    for (int r = blockIdx.x; r < a.rows; r += gridDim.x) {
      int32_t* o = a.ids + (size_t)r * a.k;
      for (int x = tid; x < a.k; x += kShThreads) o[x] = s_ids[x];
    }
  }
}

}  // namespace stk

using namespace stk;

static StkCheck check_indexer(int dtype, int h, int n, int d) {
  if (dtype != DT_F32 && dtype != DT_F16 && dtype != DT_BF16) return {false, "unsupported dtype"};
  if (h <= 0 || n <= 0 || d <= 0) return {false, "bad indexer shape"};
  if ((int64_t)h * d > kIdxMaxQ) return {false, "indexer heads * dim must be <= 4096"};
  return {true, ""};
}

static int launch_indexer(const void* iq, const void* ik, int dtype, int h, int n, int d,
                          float* scores, uint64_t* keys, hipStream_t st) {
  IndexerArgs a{iq, ik, h, n, d, 1.0 / std::sqrt((double)d), scores, keys};
  const dim3 grid((n + 15) / 16), block(256);
  const bool vec = dtype != DT_F32 && d == 128 && h == 4 &&
                   ((reinterpret_cast<uintptr_t>(iq) | reinterpret_cast<uintptr_t>(ik)) & 15) == 0;
  if (vec && dtype == DT_BF16) hipLaunchKernelGGL((k_indexer_v<bf16s, 4>), grid, block, 0, st, a);
  else if (vec) hipLaunchKernelGGL((k_indexer_v<f16s, 4>), grid, block, 0, st, a);
  else if (dtype == DT_BF16) hipLaunchKernelGGL(k_indexer<bf16s>, grid, block, 0, st, a);
  else if (dtype == DT_F16) hipLaunchKernelGGL(k_indexer<f16s>, grid, block, 0, st, a);
  else hipLaunchKernelGGL(k_indexer<float>, grid, block, 0, st, a);
  return stk_check_launch("k_indexer");
}

// The shared top-K and its rows (k_topk_shared) for n <= 16384 and
// topk <= 8192: 0 once launched, 1 when the shape is not covered.
static int launch_topk_shared(const uint64_t* keys, int n, int topk, int rows, int32_t* ids,
                              hipStream_t st) {
  if (n > kShMaxN || topk > kShMaxK) return 1;
  SharedTopkArgs a{keys, n, topk, rows, ids,
                   topk % 4 == 0 && (reinterpret_cast<uintptr_t>(ids) & 15) == 0};
  const int wgs = (rows + kShRowsPer - 1) / kShRowsPer;
  const dim3 grid(wgs < kShMaxWgs ? wgs : kShMaxWgs), block(kShThreads);
  if (n <= kShThreads) hipLaunchKernelGGL(k_topk_shared<1>, grid, block, 0, st, a);
  else if (n <= 2 * kShThreads) hipLaunchKernelGGL(k_topk_shared<2>, grid, block, 0, st, a);
  else if (n <= 4 * kShThreads) hipLaunchKernelGGL(k_topk_shared<4>, grid, block, 0, st, a);
  else if (n <= 8 * kShThreads) hipLaunchKernelGGL(k_topk_shared<8>, grid, block, 0, st, a);
  else hipLaunchKernelGGL(k_topk_shared<16>, grid, block, 0, st, a);
  return stk_check_launch("k_topk_shared");
}

extern "C" {

STK_API size_t stk_indexer_workspace_bytes(int n) {
  return n > 0 ? stk_align((size_t)n * sizeof(uint64_t)) : 0;
}

STK_API int stk_indexer_scores(const void* iq, const void* ik, int dtype, int h, int n, int d,
                               float* scores, void* workspace, size_t workspace_bytes,
                               void* stream) {
  STK_REQUIRE(check_indexer(dtype, h, n, d));
  STK_REQUIRE(iq && ik && scores, "null pointer");
  STK_REQUIRE(workspace && workspace_bytes >= stk_indexer_workspace_bytes(n),
              "workspace too small");
  return launch_indexer(iq, ik, dtype, h, n, d, scores, static_cast<uint64_t*>(workspace),
                        (hipStream_t)stream);
}

STK_API int stk_indexer_select(const void* iq, const void* ik, int dtype, int h, int n, int d,
                               int topk, int rows, float* scores, int32_t* ids, void* workspace,
                               size_t workspace_bytes, void* stream) {
  STK_REQUIRE(check_indexer(dtype, h, n, d));
  STK_REQUIRE(iq && ik && ids, "null pointer");
  STK_REQUIRE(topk >= 1 && topk <= n && rows >= 1, "bad topk or rows");
  STK_REQUIRE(workspace && workspace_bytes >= stk_indexer_workspace_bytes(n),
              "workspace too small");
  hipStream_t st = (hipStream_t)stream;
  uint64_t* keys = static_cast<uint64_t*>(workspace);
  int rc = launch_indexer(iq, ik, dtype, h, n, d, scores, keys, st);
  if (rc) return rc;
  rc = launch_topk_shared(keys, n, topk, rows, ids, st);
  if (rc <= 0) return rc;   // launched, or an error
  rc = stk_launch_topk(keys, 1, n, topk, ids, st);
  if (rc || rows == 1) return rc;
  const dim3 grid((unsigned)((topk + 255) / 256), (unsigned)(rows - 1 < 65535 ? rows - 1 : 65535));
  hipLaunchKernelGGL(k_rows_copy, grid, dim3(256), 0, st, ids, rows, topk);
  return stk_check_launch("k_rows_copy");
}

}  // extern "C"
