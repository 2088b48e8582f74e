// Hierarchical reduction of large per-block state arrays (small blocks,
// thousands of selected positions per head).
//
// Reference (6Mikao9/strict-topk-overlap) strict_topk/gqa_hierarchical.py:
//   _match_ids :10-19       -> k_match_ids (LDS position map instead of a
//                              16 x SP equality tile)
//   _packed_partials :22-52 -> k_states with the slot-skip mode
//   _groups :64-96          -> k_groups_w / k_groups (level-1 merge of 32
//                              positions)
//   _reduce :99-108         -> k_groups + k_merge
#include "common.hpp"
#include "api.hpp"

namespace stk {

constexpr int kMapN = 16384;    // block-ID range served by the LDS map
constexpr int kTileP = 32;      // positions per level-1 group (reference TILE)

struct MatchArgs {
  const void* a; int atype; int sa;
  const void* p; int ptype; int sp;
  int n;
  int32_t* slot;
};

constexpr int kMatchThreads = 1024;
constexpr int kMatchPerThread = 4;   // predicted IDs requested up front per thread

// slot[row, j] = max{p : P[row, p] == A[row, j]} or -1.  One round trip: a
// thread's selected ID and its first predicted IDs are requested before the
// map is cleared, so their loads overlap the clear.
__global__ __launch_bounds__(kMatchThreads) void k_match_ids(MatchArgs a) {
  __shared__ int32_t map[kMapN];
  const int row = blockIdx.x;
  const int j = blockIdx.y * kMatchThreads + threadIdx.x;
  if (a.n <= kMapN) {
    const int64_t aid = load_id(a.a, a.atype, (int64_t)row * a.sa + (j < a.sa ? j : 0));
    int64_t pid[kMatchPerThread];
#pragma unroll
    for (int r = 0; r < kMatchPerThread; ++r) {
      const int p = threadIdx.x + r * kMatchThreads;
      pid[r] = load_id(a.p, a.ptype, (int64_t)row * a.sp + (p < a.sp ? p : 0));
    }
    for (int i = threadIdx.x; i < a.n; i += blockDim.x) map[i] = -1;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kMatchPerThread; ++r) {
      const int p = threadIdx.x + r * kMatchThreads;
      if (p < a.sp && pid[r] >= 0 && pid[r] < a.n) atomicMax(&map[pid[r]], p);
    }
    for (int p = threadIdx.x + kMatchPerThread * kMatchThreads; p < a.sp; p += blockDim.x) {
      const int64_t id = load_id(a.p, a.ptype, (int64_t)row * a.sp + p);
      if (id >= 0 && id < a.n) atomicMax(&map[id], p);
    }
    __syncthreads();
    if (j < a.sa) a.slot[(size_t)row * a.sa + j] = (aid >= 0 && aid < a.n) ? map[aid] : -1;
  } else {
    if (j < a.sa) {
      int64_t id = load_id(a.a, a.atype, (int64_t)row * a.sa + j);
      int best = -1;
      for (int p = 0; p < a.sp; ++p)
        if (load_id(a.p, a.ptype, (int64_t)row * a.sp + p) == id) best = p;
      a.slot[(size_t)row * a.sa + j] = best;
    }
  }
}

struct GroupsArgs {
  const float* m; const float* l; const float* u;     // scratch / current [h, s]
  const float* pm; const float* pl; const float* pu;  // prediction [h, sp] (repair)
  const int32_t* slot; int shared;
  int h, s, sp, d, groups;
  float* om; float* ol; float* ou;                    // [h, groups]
};

__global__ __launch_bounds__(256) void k_groups(GroupsArgs a) {
  __shared__ float red[32];
  __shared__ float part[256 * 4];
  __shared__ float wm[kTileP];
  __shared__ const float* urow[kTileP];
  __shared__ float lval[kTileP];
  int h = blockIdx.x, g = blockIdx.y;
  int p0 = g * kTileP;
  if (threadIdx.x < kTileP) {
    int pos = p0 + threadIdx.x;
    float m = -INFINITY, l = 0.f;
    const float* ur = nullptr;
    if (pos < a.s) {
      int sl = a.slot ? a.slot[(size_t)(a.shared ? 0 : h) * a.s + pos] : -1;
      if (sl >= 0) {
        m = a.pm[(size_t)h * a.sp + sl];
        l = a.pl[(size_t)h * a.sp + sl];
        ur = a.pu + ((size_t)h * a.sp + sl) * a.d;
      } else {
        m = a.m[(size_t)h * a.s + pos];
        l = a.l[(size_t)h * a.s + pos];
        ur = a.u + ((size_t)h * a.s + pos) * a.d;
      }
    }
    wm[threadIdx.x] = m;
    lval[threadIdx.x] = l;
    urow[threadIdx.x] = ur;
  }
  __syncthreads();
  float mx = threadIdx.x < kTileP ? wm[threadIdx.x] : -INFINITY;
  mx = block_max(mx, red);
  int dt = 1;
  while (dt < a.d && dt < 256) dt <<= 1;
  int rg = 256 / dt;
  int tr = threadIdx.x / dt, td = threadIdx.x % dt;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float z = 0.f;
  for (int j = tr; j < kTileP; j += rg) {
    if (!urow[j]) continue;
    float w = wexp(wm[j], mx);
    if (td == 0) z += w * lval[j];
    for (int c = 0; c < 4; ++c) {
      int dd = td + c * dt;
      if (dd < a.d) acc[c] += w * urow[j][dd];
    }
  }
  z = block_sum(z, red);
  for (int c = 0; c < 4; ++c) part[c * 256 + threadIdx.x] = acc[c];
  __syncthreads();
  size_t orow = (size_t)h * a.groups + g;
  for (int dd = threadIdx.x; dd < a.d; dd += blockDim.x) {
    int c = dd / dt, t = dd % dt;
    float sum = 0.f;
    for (int r = 0; r < rg; ++r) sum += part[c * 256 + r * dt + t];
    a.ou[orow * a.d + dd] = sum;
  }
  if (threadIdx.x == 0) {
    a.om[orow] = mx;
    a.ol[orow] = z;
  }
}

// The same level-1 merge with one wave per (head, group of 32 positions)
// and two dependent memory round trips: (1) the group's slots (repair) and
// (2) every (m, l) and every u row of the group, all issued before any
// arithmetic.  A u row of D floats spans LPR = D / 4 lanes (16-byte loads)
// and one load instruction covers RPI = 64 / LPR rows; each row's source
// pointer and weight come from the lane that owns the position.
template <int LPR>
__global__ __launch_bounds__(256) void k_groups_w(GroupsArgs a) {
  constexpr int RPI = STK_WAVE / LPR;
  constexpr int NI = kTileP / RPI;
  static_assert(LPR >= 2 && LPR <= STK_WAVE && kTileP % RPI == 0, "row layout");
  const int waves = blockDim.x / STK_WAVE;
  const int item = blockIdx.x * waves + wave_id();
  if (item >= a.h * a.groups) return;
  const int h = item / a.groups, g = item % a.groups;
  const int lane = lane_id();
  const int pos = g * kTileP + (lane & (kTileP - 1));
  const bool in = lane < kTileP && pos < a.s;
  const int sl = a.slot ? (int)ld_or(a.slot, (int64_t)(a.shared ? 0 : h) * a.s + pos, in, -1)
                        : -1;
  const bool hit = in && sl >= 0;
  const size_t own = (size_t)h * a.s + (in ? pos : 0);
  const size_t pred = (size_t)h * a.sp + (hit ? sl : 0);
  // one address per lane, valid either way (no prediction arrays without a
  // slot table)
  float m = *(hit ? a.pm + pred : a.m + own);
  float l = *(hit ? a.pl + pred : a.l + own);
  if (!in) {
    m = -INFINITY;
    l = 0.f;
  }
  const float* row = hit ? a.pu + pred * a.d : a.u + own * a.d;
  const uint64_t rp = reinterpret_cast<uint64_t>(row);
  float4 uv[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int r = RPI * i + lane / LPR;
    const uint64_t p = ((uint64_t)(uint32_t)__shfl((int)(rp >> 32), r) << 32) |
                       (uint32_t)__shfl((int)(uint32_t)rp, r);
    uv[i] = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) +
                                              4 * (lane % LPR));
  }
  const float mx = wave_max_u(m);
  const float w = wexp(m, mx);
  const float z = wave_sum_u(w * l);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const float wr = __shfl(w, RPI * i + lane / LPR);
    // a zero weight takes nothing from its row: positions past the group's
    // end load row 0 of the scratch states, which is never written when
    // position 0 is a hit (and 0 * NaN would be NaN)
    const float4 ur = wr != 0.f ? uv[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    acc.x += wr * ur.x; acc.y += wr * ur.y; acc.z += wr * ur.z; acc.w += wr * ur.w;
  }
#pragma unroll
  for (int off = LPR; off < STK_WAVE; off <<= 1) {
    acc.x += __shfl_xor(acc.x, off); acc.y += __shfl_xor(acc.y, off);
    acc.z += __shfl_xor(acc.z, off); acc.w += __shfl_xor(acc.w, off);
  }
  const size_t orow = (size_t)h * a.groups + g;
  if (lane < LPR) *reinterpret_cast<float4*>(a.ou + orow * a.d + 4 * lane) = acc;
  if (lane == 0) {
    a.om[orow] = mx;
    a.ol[orow] = z;
  }
}

}  // namespace stk

using namespace stk;

static size_t hier_reduced_bytes(int hq, int s, int d) {
  int groups = (s + kTileP - 1) / kTileP;
  return stk_align((size_t)hq * groups * 4) * 2 + stk_align((size_t)hq * groups * d * 4);
}

static int launch_reduce(const float* m, const float* l, const float* u, const float* pm,
                         const float* pl, const float* pu, const int32_t* slot, int shared, int hq,
                         int s, int sp, int d, Carve& w, float* out, hipStream_t st) {
  int groups = (s + kTileP - 1) / kTileP;
  float* om = w.take<float>((size_t)hq * groups);
  float* ol = w.take<float>((size_t)hq * groups);
  float* ou = w.take<float>((size_t)hq * groups * d);
  GroupsArgs g{m, l, u, pm, pl, pu, slot, shared, hq, s, sp, d, groups, om, ol, ou};
  // wave-per-group kernel for D in {64, 128, 256} with 16-byte aligned rows
  const uintptr_t al = reinterpret_cast<uintptr_t>(u) | reinterpret_cast<uintptr_t>(ou) |
                       (pu ? reinterpret_cast<uintptr_t>(pu) : 0);
  const int lpr = (al & 15) == 0 && (d == 64 || d == 128 || d == 256) ? d / 4 : 0;
  const int wg = (int)(((int64_t)hq * groups + 3) / 4);
  if (lpr == 16) hipLaunchKernelGGL((k_groups_w<16>), dim3(wg), dim3(256), 0, st, g);
  else if (lpr == 32) hipLaunchKernelGGL((k_groups_w<32>), dim3(wg), dim3(256), 0, st, g);
  else if (lpr == 64) hipLaunchKernelGGL((k_groups_w<64>), dim3(wg), dim3(256), 0, st, g);
  else hipLaunchKernelGGL(k_groups, dim3(hq, groups), dim3(256), 0, st, g);
  int rc = stk_check_launch("k_groups");
  if (rc) return rc;
  return stk_launch_merge(om, ol, ou, nullptr, hq, groups, d, out, st);
}

extern "C" {

STK_API size_t stk_hier_exact_workspace_bytes(int hq, int s, int d) {
  return stk_align((size_t)hq * s * 4) * 2 + stk_align((size_t)hq * s * d * 4) +
         hier_reduced_bytes(hq, s, d);
}

// gqa_hierarchical.exact (:111-112): partials then the two-level reduction.
STK_API int stk_hier_exact(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                           int n, int b, int d, const void* selected, int sel_dtype, int sa,
                           float* out, void* workspace, size_t workspace_bytes, void* stream) {
  STK_REQUIRE(stk_check_kv(dtype, hq, hkv, n, b, d));
  STK_REQUIRE(q && k && v && selected && out, "null pointer");
  STK_REQUIRE(sa > 0, "ids must be nonempty");
  STK_REQUIRE(workspace && workspace_bytes >= stk_hier_exact_workspace_bytes(hq, sa, d),
              "workspace too small");
  hipStream_t st = (hipStream_t)stream;
  Carve w(workspace);
  float* m = w.take<float>((size_t)hq * sa);
  float* l = w.take<float>((size_t)hq * sa);
  float* u = w.take<float>((size_t)hq * sa * d);
  const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(v);
  if (stk_hier_mfma_covers(dtype, hq, hkv, b, d, align | reinterpret_cast<uintptr_t>(u))) {
    // small blocks, 8-16 query heads per KV head: the whole group on the
    // matrix cores, one state per four packs, then one LSE merge
    const int packs = (sa + 32 / b - 1) / (32 / b);
    int rc = stk_launch_hier_mfma(q, k, v, dtype, hq, hkv, n, b, d, selected, sel_dtype, sa, m, l,
                                  u, 0, st);
    if (rc) return rc;
    return stk_launch_merge(m, l, u, nullptr, hq, (packs + 3) / 4, d, out, st);
  }
  if (stk_states_comb_covers(dtype, hq, hkv, b, d, align)) {
    // small blocks: one merged state per pack of 32 / B positions, no
    // per-block states (the reference's two-level reduction, merged in
    // registers), then one LSE merge over the packs
    const int packs = (sa + 32 / b - 1) / (32 / b);
    int rc = stk_launch_states_comb(q, k, v, dtype, hq, hkv, n, b, d, selected, sel_dtype, sa,
                                    nullptr, 0, nullptr, nullptr, nullptr, 0, m, l, u, st);
    if (rc) return rc;
    return stk_launch_merge(m, l, u, nullptr, hq, (packs + 3) / 4, d, out, st);
  }
  int rc = stk_launch_states(q, k, v, dtype, hq, hkv, n, b, d, selected, sel_dtype, sa, nullptr, 0,
                             nullptr, 0, 0, nullptr, m, l, u, true, st);
  if (rc) return rc;
  return launch_reduce(m, l, u, nullptr, nullptr, nullptr, nullptr, 0, hq, sa, 0, d, w, out, st);
}

STK_API size_t stk_hier_repair_workspace_bytes(int hq, int sa, int d, int shared) {
  return stk_align((size_t)(shared ? 1 : hq) * sa * 4) + stk_align((size_t)hq * sa * 4) * 2 +
         stk_align((size_t)hq * sa * d * 4) + hier_reduced_bytes(hq, sa, d);
}

// gqa_hierarchical.repair_saved / repair_saved_shared (:115-144)
STK_API int stk_hier_repair(const void* q, const void* k, const void* v, int dtype, int hq,
                            int hkv, int n, int b, int d, const void* selected, int sel_dtype,
                            int sa, const void* predicted, int pred_dtype, int sp,
                            const float* pm, const float* pl, const float* pu, int shared,
                            float* out, void* workspace, size_t workspace_bytes, void* stream) {
  STK_REQUIRE(stk_check_kv(dtype, hq, hkv, n, b, d));
  STK_REQUIRE(q && k && v && selected && predicted && pm && pl && pu && out, "null pointer");
  STK_REQUIRE(sa > 0 && sp > 0, "ids must be nonempty");
  STK_REQUIRE(workspace && workspace_bytes >= stk_hier_repair_workspace_bytes(hq, sa, d, shared),
              "workspace too small");
  hipStream_t st = (hipStream_t)stream;
  Carve w(workspace);
  int rows = shared ? 1 : hq;
  int32_t* slot = w.take<int32_t>((size_t)rows * sa);
  float* m = w.take<float>((size_t)hq * sa);
  float* l = w.take<float>((size_t)hq * sa);
  float* u = w.take<float>((size_t)hq * sa * d);
  MatchArgs ma{selected, sel_dtype, sa, predicted, pred_dtype, sp, n, slot};
  hipLaunchKernelGGL(k_match_ids, dim3(rows, (sa + kMatchThreads - 1) / kMatchThreads),
                     dim3(kMatchThreads), 0, st, ma);
  int rc = stk_check_launch("k_match_ids");
  if (rc) return rc;
  const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(v);
  if (stk_states_comb_covers(dtype, hq, hkv, b, d, align)) {
    // the misses computed and the hits' prediction states merged per pack in
    // one launch, then one LSE merge over the packs
    const int packs = (sa + 32 / b - 1) / (32 / b);
    rc = stk_launch_states_comb(q, k, v, dtype, hq, hkv, n, b, d, selected, sel_dtype, sa, slot,
                                shared ? 1 : 0, pm, pl, pu, sp, m, l, u, st);
    if (rc) return rc;
    return stk_launch_merge(m, l, u, nullptr, hq, (packs + 3) / 4, d, out, st);
  }
  rc = stk_launch_states_skip(q, k, v, dtype, hq, hkv, n, b, d, selected, sel_dtype, sa, slot,
                              shared ? 1 : 0, m, l, u, st);
  if (rc) return rc;
  return launch_reduce(m, l, u, pm, pl, pu, slot, shared ? 1 : 0, hq, sa, sp, d, w, out, st);
}

}  // extern "C"
