// Hierarchical exact attention on the matrix cores: one wave per (KV head,
// pack of 32 tokens) computes the pack's softmax state for all G <= 16 query
// heads of the KV group with 16x16x32 MFMAs, and a workgroup merges its four
// waves' packs in LDS before writing.
//
// Reference: strict_topk/gqa_hierarchical.py:22-112 (exact: block states,
// then two merge levels).  The LSE merge is associative, so one state per
// pack of 32 / B blocks followed by one merge over the packs gives the same
// result up to FP32 rounding.
//
// Per pack (T = 32 tokens; the group's heads padded to 16 rows):
//   S^T[T x 16] = K[T x D] . Q^T[D x 16]: 2 x D/32 MFMAs on the 16-bit
//     inputs, whose products are exact in the FP32 accumulator;
//   each head's max and sum over its tokens (in-lane, then the lane groups);
//   U[16 x D] = P[16 x T] . V[T x D]: D/16 tiles, with P split into a high
//     and a low 16-bit part (two MFMAs per tile), so each weight keeps about
//     16 significant bits (the reference's P.V is FP32).
// Operand layouts (16x16x32): lane l holds row (A) / column (B) l % 16 and
// the reduction chunk 8 (l / 16) .. + 7 of A and B alike; the accumulator
// holds column l % 16, rows 4 (l / 16) .. + 3.  P's reduction index is taken
// to be the tokens the S^T accumulator already holds per lane (4g + i and
// 16 + 4g + i), and V's rows are loaded in that order; the output column c
// of tile t is dimension 8c + t, so a lane's V load is one 16-byte chunk of
// a row.  The heads share the tile when their IDs agree at the pack (an
// indexer's selection, shared by all heads); otherwise the pack is computed
// once per head with the other rows masked.
#include "api.hpp"
#include "states_tok.hpp"

namespace stk {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kHmD = 128;     // head dimension
constexpr int kHmTok = 32;    // tokens per pack
constexpr int kHmMaxG = 16;   // query heads per KV head (MFMA rows)

template <typename T> struct HmOps;
template <> struct HmOps<bf16s> {
  static constexpr float kPScale = 1.f;
  __device__ __forceinline__ static f32x4_t mma(uint4 a, uint4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  // x (finite, >= 0) = hi + lo to within 2^-16 x, as 16-bit patterns: hi is
  // x truncated (x - hi is exact in FP32), lo its rounded remainder
  __device__ __forceinline__ static void split(float x, uint32_t& hi, uint32_t& lo) {
    const uint32_t u = __float_as_uint(x);
    hi = u >> 16;
    const uint32_t r = __float_as_uint(x - __uint_as_float(u & 0xffff0000u));
    lo = (r + 0x7fffu + ((r >> 16) & 1u)) >> 16;
  }
};
template <> struct HmOps<f16s> {
  // weights (<= 1) are scaled into fp16's normal range before the split
  static constexpr float kPScale = 16384.f;
  __device__ __forceinline__ static f32x4_t mma(uint4 a, uint4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static void split(float x, uint32_t& hi, uint32_t& lo) {
    const _Float16 h = (_Float16)x;
    const _Float16 r = (_Float16)(x - (float)h);
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, r);
  }
};

__device__ __forceinline__ uint32_t word(const uint4& v, int k) {
  return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}

// BLK: per-block states [hq, s] (the block partials) instead of one merged
// state per four packs [hq, ceil(packs / 4)]
template <typename T, int BB, typename I, bool BLK>
__global__ __launch_bounds__(256) void k_hier_mfma(StatesArgs a) {
  using Ops = HmOps<T>;
  constexpr int D = kHmD, PB = kHmTok / BB, KS = D / 32, NT = D / 16;
  static_assert(kHmMaxG * PB <= 2 * STK_WAVE, "two (head, position) pairs per lane");
  const int packs = (a.s + PB - 1) / PB;
  const int wg = a.remap ? xcd_remap(blockIdx.x, gridDim.x) : blockIdx.x;
  // BLK: one wave per (KV head, pack).  Otherwise a workgroup takes four
  // consecutive packs of one KV head (a wave past the last pack computes
  // an empty state) and merges them before writing
  const int pgroups = (packs + 3) / 4;
  int kv, pack;
  if constexpr (BLK) {
    const int64_t item = (int64_t)wg * (blockDim.x / STK_WAVE) + wave_id();
    if (item >= (int64_t)a.hkv * packs) return;
    kv = (int)(item / packs);
    pack = (int)(item % packs);
  } else {
    kv = wg / pgroups;
    pack = (wg % pgroups) * 4 + wave_id();
  }
  const int G = a.hq / a.hkv, h0 = kv * G, p0 = pack * PB;
  const int lane = lane_id(), c = lane & 15, g = lane >> 4;
  const I* ids = reinterpret_cast<const I*>(a.ids);
  const T* Q = reinterpret_cast<const T*>(a.q);
  const T* K = reinterpret_cast<const T*>(a.k);
  const T* V = reinterpret_cast<const T*>(a.v);
  // ---- round trip 1: the group's IDs at the pack, two (head, position)
  // pairs per lane (pair x = lane + 64 r: head x / PB, position x % PB), and
  // the query rows as the B operand of S^T (head c, dims 32 ks + 8 g .. + 7)
  int64_t pid[2];
  bool pin[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int x = lane + STK_WAVE * r, hh = x / PB, j = x % PB;
    pin[r] = hh < G && p0 + j < a.s;
    pid[r] = ld_or(ids, (int64_t)(h0 + (hh < G ? hh : 0)) * a.s + p0 + j, pin[r], (I)-1);
  }
  uint4 qb[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    qb[ks] = c < G ? *reinterpret_cast<const uint4*>(Q + (size_t)(h0 + c) * D + 32 * ks + 8 * g)
                   : make_uint4(0u, 0u, 0u, 0u);
  // pairs with a valid block ID, as a 128-bit mask; the heads share the tile
  // when every head lists head 0's IDs at the pack
  const bool ok0 = pin[0] && pid[0] >= 0 && pid[0] < a.n;
  const bool ok1 = pin[1] && pid[1] >= 0 && pid[1] < a.n;
  const uint64_t cm0 = __ballot(ok0), cm1 = __ballot(ok1);
  const int64_t ref = __shfl(pid[0], lane % PB);
  const bool diff = (pin[0] && pid[0] != ref) || (pin[1] && pid[1] != ref);
  const bool same = __ballot(diff) == 0ull;
  const float scale = 1.0f / sqrtf((float)D);
  f32x4_t ut[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) ut[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float mrow = -INFINITY, lrow = 0.f;   // head c's max and sum
  // the pack for the heads in rmask, on head th's IDs (every shuffle and
  // MFMA below runs in all lanes)
  auto pass = [&](int th, uint32_t rmask, bool group) {
    const int xb = th * PB;   // head th's pairs lie in one 64-pair word
    const uint64_t cw = xb < STK_WAVE ? cm0 : cm1;
    const uint32_t cmask = (uint32_t)(cw >> (xb & 63)) & ((1u << PB) - 1u);
    auto id_at = [&](int j) -> int64_t {
      const int x = (xb + j) & 63;
      const int64_t v0 = __shfl(pid[0], x), v1 = __shfl(pid[1], x);
      return xb < STK_WAVE ? v0 : v1;
    };
    // ---- round trip 2: K rows 16 mt + c (A operand: dims 32 ks + 8 g ..),
    // V rows 4 g + e and 16 + 4 g + e (dims 8 c .. + 7); a position without
    // a valid ID reads block 0 and is masked
    uint4 kb[2][KS];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int tok = 16 * mt + c, j = tok / BB;
      const int64_t bid = id_at(j);
      const bool ok = (cmask >> j) & 1u;
      const T* row =
          K + (((size_t)kv * a.n + (ok ? (size_t)bid : 0)) * BB + tok % BB) * D + 8 * g;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kb[mt][ks] = *reinterpret_cast<const uint4*>(row + 32 * ks);
    }
    uint4 vb[8];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int t0 = 16 * half + 4 * g, j = t0 / BB;   // 4 tokens in one block
      const int64_t bid = id_at(j);
      const bool ok = (cmask >> j) & 1u;
      const T* blk = V + ((size_t)kv * a.n + (ok ? (size_t)bid : 0)) * BB * D + 8 * c;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        vb[4 * half + e] = *reinterpret_cast<const uint4*>(blk + (size_t)((t0 + e) % BB) * D);
    }
    // ---- S^T = K . Q^T
    f32x4_t st[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      st[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) st[mt] = Ops::mma(kb[mt][ks], qb[ks], st[mt]);
    }
    // head c's scores at tokens 4 g + e (e < 4) and 16 + 4 g + e - 4
    const bool on = (rmask >> c) & 1u;
    float sv[8], mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int tok = 16 * (e / 4) + 4 * g + (e & 3), j = tok / BB;
      const bool ok = on && ((cmask >> j) & 1u);
      sv[e] = ok ? st[e / 4][e & 3] * scale : -INFINITY;
      mx = fmaxf(mx, sv[e]);
    }
    if constexpr (BLK) {
      // ---- per-block states.  Token k(g, e) lies in block
      // (16 (e / 4) + 4 g + (e & 3)) / B: each half of a lane's tokens is one
      // block (B = 8: shared with lane group g ^ 1), so a block's max and sum
      // stay in the lane (one exchange for B = 8)
      float p[8], mb[2], lb[2];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        float x = fmaxf(fmaxf(sv[4 * hf], sv[4 * hf + 1]), fmaxf(sv[4 * hf + 2], sv[4 * hf + 3]));
        if constexpr (BB == 8) x = fmaxf(x, __shfl_xor(x, 16));
        float y = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          p[4 * hf + e] = wexp(sv[4 * hf + e], x);
          y += p[4 * hf + e];
        }
        if constexpr (BB == 8) y += __shfl_xor(y, 16);
        mb[hf] = x;
        lb[hf] = y;
      }
      // m and l from the lanes of their head (column c)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int j = (16 * hf + 4 * g) / BB;
        if (on && p0 + j < a.s && (BB == 4 || (g & 1) == 0)) {
          const int64_t row = (int64_t)(h0 + c) * a.s + p0 + j;
          a.m[row] = mb[hf];
          a.l[row] = lb[hf];
        }
      }
      uint32_t ah[4], al[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t h0w, l0w, h1w, l1w;
        Ops::split(p[2 * q] * Ops::kPScale, h0w, l0w);
        Ops::split(p[2 * q + 1] * Ops::kPScale, h1w, l1w);
        ah[q] = h0w | (h1w << 16);
        al[q] = l0w | (l1w << 16);
      }
      uint4 bv[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int sh = 16 * (t & 1);
        uint32_t bw[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          bw[q] = ((word(vb[2 * q], t / 2) >> sh) & 0xffffu) |
                  (((word(vb[2 * q + 1], t / 2) >> sh) & 0xffffu) << 16);
        bv[t] = make_uint4(bw[0], bw[1], bw[2], bw[3]);
      }
      // the block of P's words q (elements 2q, 2q + 1)
      auto blk_of = [&](int q) { return (16 * (q / 2) + 4 * g + 2 * (q & 1)) / BB; };
      constexpr float inv = 1.f / Ops::kPScale;
      auto block_u = [&](const uint32_t (&wh)[4], const uint32_t (&wl)[4], int keep,
                         f32x4_t (&uj)[NT]) {
        uint32_t kh[4], kl[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          kh[q] = blk_of(q) == keep ? wh[q] : 0u;
          kl[q] = blk_of(q) == keep ? wl[q] : 0u;
        }
        const uint4 xh = make_uint4(kh[0], kh[1], kh[2], kh[3]);
        const uint4 xl = make_uint4(kl[0], kl[1], kl[2], kl[3]);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          uj[t] = Ops::mma(xh, bv[t], f32x4_t{0.f, 0.f, 0.f, 0.f});
          uj[t] = Ops::mma(xl, bv[t], uj[t]);
        }
      };
      auto store_u = [&](int64_t row, const f32x4_t (&uj)[NT], int i) {
        float4* dst = reinterpret_cast<float4*>(a.u + row * D + 8 * c);
        dst[0] = make_float4(uj[0][i] * inv, uj[1][i] * inv, uj[2][i] * inv, uj[3][i] * inv);
        dst[1] = make_float4(uj[4][i] * inv, uj[5][i] * inv, uj[6][i] * inv, uj[7][i] * inv);
      };
      f32x4_t uj[NT];
      if (group) {
        // the group's heads share the tokens: block j's U for all heads at
        // once (P restricted to block j); output rows are heads 4 g + i
        for (int j = 0; j < PB; ++j) {
          block_u(ah, al, j, uj);
          if (p0 + j < a.s) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int hr = 4 * g + i;
              if (hr < G) store_u((int64_t)(h0 + hr) * a.s + p0 + j, uj, i);
            }
          }
        }
      } else {
        // one head: the MFMA rows become the pack's blocks.  Lane (c, g)
        // takes head th's words (lane 16 g + th) and keeps those of block c;
        // output rows are blocks 4 g + i
        uint32_t th_h[4], th_l[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          th_h[q] = __shfl(ah[q], 16 * g + th);
          th_l[q] = __shfl(al[q], 16 * g + th);
        }
        block_u(th_h, th_l, c, uj);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * g + i;
          if (r < PB && p0 + r < a.s) store_u((int64_t)(h0 + th) * a.s + p0 + r, uj, i);
        }
      }
      return;
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    float p[8], ls = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = wexp(sv[e], mx);
      ls += p[e];
    }
    ls += __shfl_xor(ls, 16);
    ls += __shfl_xor(ls, 32);
    // every head is in exactly one pass
    if (on) {
      mrow = mx;
      lrow = ls;
    }
    // ---- U += P . V (P's rows are off for the heads outside rmask)
    uint32_t ah[4], al[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t h0w, l0w, h1w, l1w;
      Ops::split(p[2 * q] * Ops::kPScale, h0w, l0w);
      Ops::split(p[2 * q + 1] * Ops::kPScale, h1w, l1w);
      ah[q] = h0w | (h1w << 16);
      al[q] = l0w | (l1w << 16);
    }
    const uint4 pah = make_uint4(ah[0], ah[1], ah[2], ah[3]);
    const uint4 pal = make_uint4(al[0], al[1], al[2], al[3]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int sh = 16 * (t & 1);
      uint32_t bw[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        bw[q] = ((word(vb[2 * q], t / 2) >> sh) & 0xffffu) |
                (((word(vb[2 * q + 1], t / 2) >> sh) & 0xffffu) << 16);
      const uint4 bv = make_uint4(bw[0], bw[1], bw[2], bw[3]);
      ut[t] = Ops::mma(pah, bv, ut[t]);
      ut[t] = Ops::mma(pal, bv, ut[t]);
    }
  };
  const uint32_t all = (1u << G) - 1u;
  if (same) {
    pass(0, all, true);
  } else {
    for (int th = 0; th < G; ++th) pass(th, 1u << th, false);
  }
  if constexpr (BLK) return;
  // ---- the pack's state per head to LDS: lane (c, g) holds heads 4 g + i,
  // dimensions 8 c .. 8 c + 7 (tile t = dimension 8 c + t)
  __shared__ __align__(16) float s_u[4][kHmMaxG][D];
  __shared__ float s_m[4][kHmMaxG], s_l[4][kHmMaxG];
  const int w = wave_id();
  constexpr float inv = 1.f / Ops::kPScale;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hr = 4 * g + i;
    const float mi = __shfl(mrow, hr), li = __shfl(lrow, hr);
    float4* dst = reinterpret_cast<float4*>(&s_u[w][hr][8 * c]);
    dst[0] = make_float4(ut[0][i] * inv, ut[1][i] * inv, ut[2][i] * inv, ut[3][i] * inv);
    dst[1] = make_float4(ut[4][i] * inv, ut[5][i] * inv, ut[6][i] * inv, ut[7][i] * inv);
    if (c == 0) {
      s_m[w][hr] = mi;
      s_l[w][hr] = li;
    }
  }
  __syncthreads();
  // ---- one state per (head, four packs): wave w merges heads 4 w .. 4 w + 3,
  // lane l dimensions 2 l, 2 l + 1
  const int grp = wg % pgroups;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hr = 4 * w + i;
    if (hr >= G) break;
    float M = -INFINITY;
#pragma unroll
    for (int x = 0; x < 4; ++x) M = fmaxf(M, s_m[x][hr]);
    float L = 0.f, u0 = 0.f, u1 = 0.f;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const float f = wexp(s_m[x][hr], M);   // 0 for an empty pack
      const float2 ux = *reinterpret_cast<const float2*>(&s_u[x][hr][2 * lane]);
      L += f * s_l[x][hr];
      u0 += f * ux.x;
      u1 += f * ux.y;
    }
    const int64_t row = (int64_t)(h0 + hr) * pgroups + grp;
    *reinterpret_cast<float2*>(a.u + row * D + 2 * lane) = make_float2(u0, u1);
    if (lane == 0) {
      a.m[row] = M;
      a.l[row] = L;
    }
  }
}

}  // namespace
}  // namespace stk

using namespace stk;

bool stk_hier_mfma_covers(int dtype, int hq, int hkv, int b, int d, uintptr_t align) {
  if (dtype != DT_BF16 && dtype != DT_F16) return false;
  if (d != kHmD || (b != 4 && b != 8) || (align & 15) != 0) return false;
  if (hkv <= 0 || hq % hkv != 0) return false;
  const int G = hq / hkv;
  return G >= 8 && G <= kHmMaxG;
}

int stk_launch_hier_mfma(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                         int n, int b, int d, const void* ids, int itype, int s, float* m,
                         float* l, float* u, int blocks, hipStream_t st) {
  const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(u);
  if (!stk_hier_mfma_covers(dtype, hq, hkv, b, d, align) || s <= 0) return STK_EINVAL;
  StatesArgs a{};
  a.q = q; a.k = k; a.v = v; a.ids = ids; a.itype = itype;
  a.hq = hq; a.hkv = hkv; a.n = n; a.b = b; a.d = d; a.s = s;
  a.m = m; a.l = l; a.u = u;
  const int packs = (s + kHmTok / b - 1) / (kHmTok / b);
  // block mode: one wave per (KV head, pack); merged mode: one workgroup per
  // (KV head, four packs)
  const int64_t items = (int64_t)hkv * packs;
  const int grid = blocks ? (int)((items + 3) / 4) : hkv * ((packs + 3) / 4);
  a.remap = grid >= 8 ? 1 : 0;
  const bool i64 = itype == IT_I64;
#define STK_HM1(TT, BBV, IT)                                                                \
  do {                                                                                      \
    if (blocks)                                                                             \
      hipLaunchKernelGGL((k_hier_mfma<TT, BBV, IT, true>), dim3(grid), dim3(256), 0, st, a); \
    else                                                                                    \
      hipLaunchKernelGGL((k_hier_mfma<TT, BBV, IT, false>), dim3(grid), dim3(256), 0, st, a); \
  } while (0)
#define STK_HM(TT, BBV)             \
  do {                              \
    if (i64)                        \
      STK_HM1(TT, BBV, int64_t);    \
    else                            \
      STK_HM1(TT, BBV, int32_t);    \
  } while (0)
  if (dtype == DT_BF16) {
    if (b == 4) STK_HM(bf16s, 4);
    else STK_HM(bf16s, 8);
  } else {
    if (b == 4) STK_HM(f16s, 4);
    else STK_HM(f16s, 8);
  }
#undef STK_HM
#undef STK_HM1
  return stk_check_launch("k_hier_mfma");
}
