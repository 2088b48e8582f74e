// Min/max query-sign bound scorer plus exact top-K selection.
//
// Reference: strict_topk/selector.py:8-20,30-50 (_score, block_scores,
// select_blocks) and strict_topk/gqa.py:15-26,365-381 (_bound_score,
// select_blocks), which end in torch.topk(sorted=False).
//
// Contract: score[h,n] = sum_d q_d * (q_d >= 0 ? hi : lo)[h/G, n, d] in FP64.
// Products are exact; 16 lanes share a block, lane c summing dims
// 64*j + 4*c + t (j ascending, t = 0..3) from +0.0, then lanes combine with an
// xor butterfly (8, 4, 2, 1).  The top K are the K largest (score, -index)
// pairs, i.e. ties go to the lower block index; IDs are written in
// (score desc, index asc) order.
//
// Launch structure (MI355X): k_score_sort spreads the HBM-bound metadata
// stream over (KV head x head subgroup x chunk) workgroups; every workgroup
// scores CH blocks for GS query heads sharing one KV head (lo/hi read once
// per subgroup), bitonic-sorts each head's chunk in LDS and keeps its best KP.
// k_topk_merge then merges the per-chunk sorted lists of a row with a tree of
// bitonic half-cleaners.
#include "common.hpp"
#include "api.hpp"

namespace stk {

constexpr int kSortElems = 4096;   // GS * CHP per scoring workgroup
constexpr int kMergeElems = 8192;  // elements resident in the merge workgroup
constexpr int kMaxGS = 16;
constexpr int kQElems = 4096;      // GS * D query values staged in LDS

__device__ __forceinline__ uint64_t score_key(double s) {
  if (s != s) return 0ull;
  if (s == 0.0) s = 0.0;
  uint64_t b = (uint64_t)__double_as_longlong(s);
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}

__device__ __forceinline__ bool better(uint64_t ka, uint32_t ia, uint64_t kb, uint32_t ib) {
  return ka > kb || (ka == kb && ia < ib);
}

struct ScoreArgs {
  const void* q; int qtype;
  const float* lo; const float* hi;
  int hq, hkv, n, d;
  int gs;        // heads per workgroup
  int ch;        // blocks per chunk
  int chp;       // next pow2 of ch
  int kp;        // list length kept per chunk (pow2)
  int nchunks;
  float* scores;     // optional FP32 [hq, n]
  uint64_t* wkey;    // optional [hq, nchunks, kp]
  uint32_t* widx;
};

template <typename Q>
__device__ __forceinline__ float qval(const void* q, int64_t i) {
  return cvt(reinterpret_cast<const Q*>(q)[i]);
}

template <typename Q, bool SORT>
__global__ __launch_bounds__(256) void k_score_sort(ScoreArgs a) {
  __shared__ float qs[kQElems];   // per-head query rows (FP32 copies)
  __shared__ uint64_t skey[kSortElems];
  __shared__ uint32_t sidx[kSortElems];
  const int G = a.hq / a.hkv;
  const int hg = (G + a.gs - 1) / a.gs;
  const int kv = blockIdx.x / hg;
  const int g0 = (blockIdx.x % hg) * a.gs;
  const int gs = min(a.gs, G - g0);
  const int h0 = kv * G + g0;
  const int chunk = blockIdx.y;
  const int n0 = chunk * a.ch;
  const int nend = min(a.n, n0 + a.ch);
  for (int i = threadIdx.x; i < gs * a.d; i += blockDim.x)
    qs[i] = qval<Q>(a.q, (int64_t)h0 * a.d + i);
  if (SORT)
    for (int i = threadIdx.x; i < gs * a.chp; i += blockDim.x) {
      skey[i] = 0ull;
      sidx[i] = 0xffffffffu;
    }
  __syncthreads();
  const int lane16 = threadIdx.x & 15;
  const int slot = threadIdx.x >> 4;          // 16 blocks per pass of 256 threads
  const int passes = (a.d + 63) / 64;
  const bool vec4 = (a.d & 3) == 0;
  const int iters = (a.ch + 15) / 16;
  for (int it = 0; it < iters; ++it) {
    // every lane of a 16-group takes part in the butterfly, valid or not
    int nb = n0 + it * 16 + slot;
    bool valid = nb < nend && it * 16 + slot < a.ch;
    double acc[kMaxGS];
#pragma unroll
    for (int g = 0; g < kMaxGS; ++g) acc[g] = 0.0;
    if (valid) {
      const float* lrow = a.lo + ((size_t)kv * a.n + nb) * a.d;
      const float* hrow = a.hi + ((size_t)kv * a.n + nb) * a.d;
      for (int j = 0; j < passes; ++j) {
        int d0 = 64 * j + 4 * lane16;
        float lv[4], hv[4];
        if (vec4 && d0 + 3 < a.d) {
          float4 l4 = *reinterpret_cast<const float4*>(lrow + d0);
          float4 h4 = *reinterpret_cast<const float4*>(hrow + d0);
          lv[0] = l4.x; lv[1] = l4.y; lv[2] = l4.z; lv[3] = l4.w;
          hv[0] = h4.x; hv[1] = h4.y; hv[2] = h4.z; hv[3] = h4.w;
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            lv[t] = d0 + t < a.d ? lrow[d0 + t] : 0.f;
            hv[t] = d0 + t < a.d ? hrow[d0 + t] : 0.f;
          }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          int dd = d0 + t;
          if (dd < a.d) {
#pragma unroll
            for (int g = 0; g < kMaxGS; ++g) {
              if (g < gs) {
                float qv = qs[g * a.d + dd];
                double b = qv >= 0.f ? (double)hv[t] : (double)lv[t];
                acc[g] = acc[g] + (double)qv * b;   // exact product, one rounding
              }
            }
          }
        }
      }
    }
    for (int g = 0; g < gs; ++g) {
      double v = acc[g];
      v = v + __shfl_xor(v, 8);
      v = v + __shfl_xor(v, 4);
      v = v + __shfl_xor(v, 2);
      v = v + __shfl_xor(v, 1);
      if (valid && lane16 == 0) {
        if (v == 0.0) v = 0.0;
        int h = h0 + g;
        if (a.scores) a.scores[(size_t)h * a.n + nb] = (float)v;
        if (SORT) {
          skey[g * a.chp + (nb - n0)] = score_key(v);
          sidx[g * a.chp + (nb - n0)] = (uint32_t)nb;
        }
      }
    }
  }
  if (!SORT) return;
  __syncthreads();
  // bitonic sort of each head's chp entries, descending by (key, -idx)
  const int total = gs * a.chp;
  for (int k = 2; k <= a.chp; k <<= 1) {
    for (int jj = k >> 1; jj > 0; jj >>= 1) {
      for (int i = threadIdx.x; i < total; i += blockDim.x) {
        int li = i & (a.chp - 1);
        int p = li ^ jj;
        if (p > li) {
          int base = i - li;
          uint64_t k1 = skey[base + li], k2 = skey[base + p];
          uint32_t i1 = sidx[base + li], i2 = sidx[base + p];
          bool desc = (li & k) == 0;
          bool swap = desc ? better(k2, i2, k1, i1) : better(k1, i1, k2, i2);
          if (swap) {
            skey[base + li] = k2; skey[base + p] = k1;
            sidx[base + li] = i2; sidx[base + p] = i1;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < gs * a.kp; i += blockDim.x) {
    int g = i / a.kp, r = i % a.kp;
    size_t o = ((size_t)(h0 + g) * a.nchunks + chunk) * a.kp + r;
    if (r < a.chp) {
      a.wkey[o] = skey[g * a.chp + r];
      a.widx[o] = sidx[g * a.chp + r];
    } else {
      a.wkey[o] = 0ull;
      a.widx[o] = 0xffffffffu;
    }
  }
}

struct MergeTopArgs {
  const uint64_t* wkey; const uint32_t* widx;
  int nchunks, kp, k;
  int32_t* ids;
};

// Sorted-list tree merge per row.  LDS holds `cap` lists of kp entries; the
// running best list stays in list 0 between batches.
__global__ __launch_bounds__(1024) void k_topk_merge(MergeTopArgs a) {
  __shared__ uint64_t key[kMergeElems];
  __shared__ uint32_t idx[kMergeElems];
  const int h = blockIdx.x;
  const int kp = a.kp;
  const int cap = kMergeElems / kp;      // lists resident (pow2, >= 2)
  const uint64_t* rk = a.wkey + (size_t)h * a.nchunks * kp;
  const uint32_t* ri = a.widx + (size_t)h * a.nchunks * kp;
  int next = 0;
  bool have = false;
  while (next < a.nchunks || !have) {
    int first = have ? 1 : 0;
    int take = min(cap - first, a.nchunks - next);
    int lists = first + take;
    int lp = 1;
    while (lp < lists) lp <<= 1;
    for (int i = threadIdx.x; i < (lp - first) * kp; i += blockDim.x) {
      int li = first + i / kp, r = i % kp;
      int src = next + (li - first);
      if (li < lists) {
        key[li * kp + r] = rk[(size_t)src * kp + r];
        idx[li * kp + r] = ri[(size_t)src * kp + r];
      } else {
        key[li * kp + r] = 0ull;
        idx[li * kp + r] = 0xffffffffu;
      }
    }
    next += take;
    have = true;
    __syncthreads();
    for (int stride = 1; stride < lp; stride <<= 1) {
      int pairs = lp / (2 * stride);
      // half-cleaner: a[i] vs b[kp-1-i]
      for (int i = threadIdx.x; i < pairs * kp; i += blockDim.x) {
        int p = i / kp, r = i % kp;
        int la = (2 * p) * stride, lb = la + stride;
        int ia = la * kp + r, ib = lb * kp + (kp - 1 - r);
        if (better(key[ib], idx[ib], key[ia], idx[ia])) {
          key[ia] = key[ib];
          idx[ia] = idx[ib];
        }
      }
      __syncthreads();
      // bitonic merge of each surviving list into descending order
      for (int jj = kp >> 1; jj > 0; jj >>= 1) {
        for (int i = threadIdx.x; i < pairs * kp; i += blockDim.x) {
          int p = i / kp, r = i % kp;
          int q = r ^ jj;
          if (q > r) {
            int base = (2 * p) * stride * kp;
            uint64_t k1 = key[base + r], k2 = key[base + q];
            uint32_t i1 = idx[base + r], i2 = idx[base + q];
            if (better(k2, i2, k1, i1)) {
              key[base + r] = k2; key[base + q] = k1;
              idx[base + r] = i2; idx[base + q] = i1;
            }
          }
        }
        __syncthreads();
      }
    }
    if (next >= a.nchunks) break;
  }
  for (int i = threadIdx.x; i < a.k; i += blockDim.x) a.ids[(size_t)h * a.k + i] = (int32_t)idx[i];
}

static int pow2ceil(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

struct SelectPlan {
  int gs, ch, chp, kp, nchunks, hg;
};

static SelectPlan plan_select(int hq, int hkv, int n, int d, int topk) {
  SelectPlan p{};
  int G = hq / hkv;
  p.kp = pow2ceil(topk < 1 ? 1 : topk);
  p.ch = p.kp > 64 ? p.kp : 64;
  if (p.ch > n) p.ch = n;
  p.chp = pow2ceil(p.ch);
  if (p.chp < p.kp) p.chp = p.kp;   // keeps the sort length >= kept length
  int gs = kSortElems / p.chp;
  if (gs > kMaxGS) gs = kMaxGS;
  if (gs > kQElems / d) gs = kQElems / d;
  if (gs > G) gs = G;
  if (gs < 1) gs = 1;
  p.gs = gs;
  p.hg = (G + gs - 1) / gs;
  p.nchunks = (n + p.ch - 1) / p.ch;
  return p;
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

template <bool SORT>
static void launch_score(ScoreArgs& a, int qtype, dim3 grid, hipStream_t st) {
  if (qtype == DT_BF16)
    hipLaunchKernelGGL((k_score_sort<bf16s, SORT>), grid, dim3(256), 0, st, a);
  else if (qtype == DT_F16)
    hipLaunchKernelGGL((k_score_sort<f16s, SORT>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((k_score_sort<float, SORT>), grid, dim3(256), 0, st, a);
}

extern "C" {

STK_API int stk_block_scores(const void* q, int q_dtype, const float* lo, const float* hi, int hq,
                             int hkv, int n, int d, float* scores, void* stream) {
  STK_REQUIRE(check_select(q_dtype, hq, hkv, n, d));
  STK_REQUIRE(q && lo && hi && scores, "null pointer");
  SelectPlan p = plan_select(hq, hkv, n, d, 1);
  int G = hq / hkv;
  ScoreArgs a{};
  a.q = q; a.qtype = q_dtype; a.lo = lo; a.hi = hi;
  a.hq = hq; a.hkv = hkv; a.n = n; a.d = d;
  a.gs = G < kMaxGS ? G : kMaxGS;
  if (a.gs > kQElems / d) a.gs = kQElems / d;
  a.ch = 64; a.chp = 64; a.kp = 1;
  a.nchunks = (n + 63) / 64;
  a.scores = scores;
  int hg = (G + a.gs - 1) / a.gs;
  (void)p;
  launch_score<false>(a, q_dtype, dim3(hkv * hg, a.nchunks), (hipStream_t)stream);
  return stk_check_launch("k_score_sort");
}

STK_API size_t stk_select_workspace_bytes(int hq, int hkv, int n, int d, int topk) {
  if (hq <= 0 || hkv <= 0 || n <= 0 || d <= 0 || topk <= 0) return 0;
  SelectPlan p = plan_select(hq, hkv, n, d, topk);
  size_t elems = (size_t)hq * p.nchunks * p.kp;
  return stk_align(elems * 8) + stk_align(elems * 4);
}

STK_API int stk_select_blocks(const void* q, int q_dtype, const float* lo, const float* hi, int hq,
                              int hkv, int n, int d, int topk, float* scores, int32_t* ids,
                              void* workspace, size_t workspace_bytes, void* stream) {
  STK_REQUIRE(check_select(q_dtype, hq, hkv, n, d));
  STK_REQUIRE(q && lo && hi && ids, "null pointer");
  STK_REQUIRE(topk >= 1 && topk <= n, "selected index k out of range");
  STK_REQUIRE(pow2ceil(topk) <= kMergeElems / 2, "topk above 4096 is not supported");
  STK_REQUIRE(workspace && workspace_bytes >= stk_select_workspace_bytes(hq, hkv, n, d, topk),
              "workspace too small");
  SelectPlan p = plan_select(hq, hkv, n, d, topk);
  Carve w(workspace);
  size_t elems = (size_t)hq * p.nchunks * p.kp;
  ScoreArgs a{};
  a.q = q; a.qtype = q_dtype; a.lo = lo; a.hi = hi;
  a.hq = hq; a.hkv = hkv; a.n = n; a.d = d;
  a.gs = p.gs; a.ch = p.ch; a.chp = p.chp; a.kp = p.kp; a.nchunks = p.nchunks;
  a.scores = scores;
  a.wkey = w.take<uint64_t>(elems);
  a.widx = w.take<uint32_t>(elems);
  hipStream_t st = (hipStream_t)stream;
  launch_score<true>(a, q_dtype, dim3(hkv * p.hg, p.nchunks), st);
  int rc = stk_check_launch("k_score_sort");
  if (rc) return rc;
  MergeTopArgs m{a.wkey, a.widx, p.nchunks, p.kp, topk, ids};
  hipLaunchKernelGGL(k_topk_merge, dim3(hq), dim3(1024), 0, st, m);
  return stk_check_launch("k_topk_merge");
}

}  // extern "C"
