// Token-parallel softmax tile for one (query head(s), KV block) pair, built
// for CDNA4 wave64.
//
// Q.K: four lanes share a token row.  Lane (slot, p) holds NCH 16-byte chunks
// of the row, chunk c covering dims (c*4 + p)*EPC .. +EPC-1, so the four
// lanes of a slot read 64 contiguous bytes per instruction; 16 token slots
// per pass, UP passes per chunk of tokens.  16-bit inputs use the packed
// dot2 instruction (bf16 x bf16 and f16 x f16 products are exact in FP32)
// against the query held as packed pairs; the four partial dots combine with
// two xor shuffles inside the quad.
//
// P.V: lanes own dims (lane*DPL .. +DPL-1, one 2/4/8-byte access per token
// row, 256 contiguous bytes per wave instruction); each token's weight is
// broadcast from the lane that computed it (readlane) and accumulated with
// FP32 FMAs, so no cross-lane reduction of the value vector is needed.  The
// running state (m, l, acc) is wave-uniform in m and l.
//
// Supported shapes: D = 4 * NCH * EPC with D a multiple of 64 (DPL >= 1)
// and B a multiple of 16 (whole chunks); every other shape uses the
// generic Tile.
#pragma once

#include "attn.hpp"

namespace stk {

template <typename T> struct Elem;
template <> struct Elem<bf16s> {
  __device__ __forceinline__ static float dot(uint32_t k, uint32_t q, float acc) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, k), __builtin_bit_cast(v2, q),
                                           acc, false);
  }
  __device__ __forceinline__ static float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ __forceinline__ static float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
};
template <> struct Elem<f16s> {
  __device__ __forceinline__ static float dot(uint32_t k, uint32_t q, float acc) {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, k), __builtin_bit_cast(v2, q), acc,
                                  false);
  }
  __device__ __forceinline__ static float lo(uint32_t w) { return cvt(f16s{uint16_t(w & 0xffffu)}); }
  __device__ __forceinline__ static float hi(uint32_t w) { return cvt(f16s{uint16_t(w >> 16)}); }
};
template <> struct Elem<float> {
  __device__ __forceinline__ static float dot(uint32_t k, uint32_t q, float acc) {
    return fmaf(__uint_as_float(k), __uint_as_float(q), acc);
  }
};

template <typename T, int NCH, int UP>
struct TokTile {
  static constexpr int EPC = 16 / (int)sizeof(T);   // elements per 16-byte chunk
  static constexpr int LPT = 4;                      // lanes per token row (Q.K)
  static constexpr int TPP = STK_WAVE / LPT;         // token slots per pass
  static constexpr int D = LPT * NCH * EPC;
  static constexpr int DPL = D / STK_WAVE;           // P.V dims per lane
  static constexpr int QW = NCH * 4;                 // query words per lane
  static constexpr int CH = TPP * UP;                // tokens per chunk
  static constexpr int VW = (DPL * (int)sizeof(T) + 3) / 4;   // value words per token
  static_assert(DPL >= 1 && D % STK_WAVE == 0, "D must be a multiple of 64");

  int slot, part;
  __device__ __forceinline__ void init() {
    slot = lane_id() / LPT;
    part = lane_id() % LPT;
  }
  __device__ __forceinline__ int kdim(int c) const { return (c * LPT + part) * EPC; }

  // query row in the Q.K lane layout (raw words)
  __device__ __forceinline__ void load_q(const T* q, uint32_t* qw) const {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      uint4 x = *reinterpret_cast<const uint4*>(q + kdim(c));
      qw[4 * c + 0] = x.x; qw[4 * c + 1] = x.y; qw[4 * c + 2] = x.z; qw[4 * c + 3] = x.w;
    }
  }

  // K rows of one chunk (tokens t0 + slot + TPP*u) and V rows (tokens t0 .. t0+CH-1)
  // of the block at kb/vb.  The chunk lies inside the block (the token tile
  // is only used when CH divides B), so every row address is a constant
  // offset from one base per lane and no address needs a clamp.
  __device__ __forceinline__ void load(const T* kb, const T* vb, int t0,
                                       uint32_t (&kw)[UP][QW], uint32_t (&vw)[CH][VW]) const {
    const T* krow = kb + (size_t)(t0 + slot) * D;
#pragma unroll
    for (int u = 0; u < UP; ++u) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        uint4 x = *reinterpret_cast<const uint4*>(krow + (size_t)TPP * u * D + kdim(c));
        kw[u][4 * c + 0] = x.x; kw[u][4 * c + 1] = x.y; kw[u][4 * c + 2] = x.z;
        kw[u][4 * c + 3] = x.w;
      }
    }
    const T* vrow = vb + (size_t)t0 * D + lane_id() * DPL;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const T* row = vrow + (size_t)i * D;
      if constexpr (DPL * sizeof(T) == 2) {
        vw[i][0] = *reinterpret_cast<const uint16_t*>(row);
      } else if constexpr (DPL * sizeof(T) == 4) {
        vw[i][0] = *reinterpret_cast<const uint32_t*>(row);
      } else if constexpr (DPL * sizeof(T) == 8) {
        uint2 x = *reinterpret_cast<const uint2*>(row);
        vw[i][0] = x.x; vw[i][1] = x.y;
      } else {
        uint4 x = *reinterpret_cast<const uint4*>(row);
        vw[i][0] = x.x; vw[i][1] = x.y; vw[i][2] = x.z; vw[i][3] = x.w;
      }
    }
  }

  // value vector of token i of the chunk as FP32 (this lane's DPL dims)
  __device__ __forceinline__ void vals(const uint32_t (&vw)[CH][VW], int i, float* out) const {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int e = 0; e < DPL; ++e) out[e] = __uint_as_float(vw[i][e]);
    } else {
#pragma unroll
      for (int e = 0; e < DPL; ++e)
        out[e] = (e & 1) ? Elem<T>::hi(vw[i][e / 2]) : Elem<T>::lo(vw[i][e / 2]);
    }
  }

  // scaled logits of the chunk's tokens in this lane's slot (-inf past B)
  __device__ __forceinline__ void scores(const uint32_t* qw, const uint32_t (&kw)[UP][QW], int t0,
                                         int B, float scale, float* s) const {
#pragma unroll
    for (int u = 0; u < UP; ++u) {
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < QW; ++w) acc = Elem<T>::dot(kw[u][w], qw[w], acc);
      acc = quad_sum(acc);
      int t = t0 + slot + TPP * u;
      s[u] = t < B ? acc * scale : -INFINITY;
    }
  }

  // Online-softmax update of (m, l, acc) with one chunk whose scaled logits
  // s (this lane's slot, scores()) are known.  FIXED keeps m as the exponent
  // frame (no rescaling; the caller guarantees it).  ABS also accumulates
  // sum |w * v| (low-group envelope).  MASKV: tokens vlim .. CH-1 of the
  // chunk hold no data (their logits must be -inf); their values are taken
  // as zero, so whatever the memory holds there (NaN included) adds nothing.
  template <bool FIXED, bool ABS, bool MASKV = false>
  __device__ __forceinline__ void accumulate(const float (&s)[UP], const uint32_t (&vw)[CH][VW],
                                             float& m, float& l, float* acc,
                                             float* aacc = nullptr, int vlim = CH) const {
    if constexpr (!FIXED) {
      float cm = s[0];
#pragma unroll
      for (int u = 1; u < UP; ++u) cm = fmaxf(cm, s[u]);
      cm = wave_max_u(cm);
      float nm = fmaxf(m, cm);
      if (nm > m) {
        float alpha = wexp(m, nm);
        l *= alpha;
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[e] *= alpha;
        m = nm;
      }
    }
    float w[UP];
#pragma unroll
    for (int u = 0; u < UP; ++u) w[u] = wexp(s[u], m);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int u = i / TPP, src = (i % TPP) * LPT;
      float wt = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w[u]), src));
      float v[DPL];
      vals(vw, i, v);
      if constexpr (MASKV) {
#pragma unroll
        for (int e = 0; e < DPL; ++e) v[e] = i < vlim ? v[e] : 0.f;
      }
      l += wt;
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        float x = wt * v[e];
        acc[e] += x;
        if constexpr (ABS) aacc[e] += fabsf(x);
      }
    }
  }

  // scores() then accumulate() for one chunk
  template <bool FIXED, bool ABS>
  __device__ __forceinline__ void update(const uint32_t* qw, const uint32_t (&kw)[UP][QW],
                                         const uint32_t (&vw)[CH][VW], int t0, int B,
                                         float scale, float& m, float& l, float* acc,
                                         float* aacc = nullptr) const {
    float s[UP];
    scores(qw, kw, t0, B, scale, s);
    accumulate<FIXED, ABS>(s, vw, m, l, acc, aacc);
  }

  // update() for a chunk of a partly filled block: tokens t0 + j with
  // t0 + j >= valid hold no data (no weight, values taken as zero)
  __device__ __forceinline__ void update_part(const uint32_t* qw, const uint32_t (&kw)[UP][QW],
                                              const uint32_t (&vw)[CH][VW], int t0, int valid,
                                              float scale, float& m, float& l,
                                              float* acc) const {
    float s[UP];
    scores(qw, kw, t0, valid, scale, s);
    accumulate<false, false, true>(s, vw, m, l, acc, nullptr, valid - t0);
  }

  // this lane's DPL dims of a D-vector
  __device__ __forceinline__ void store(float* dst, const float* acc, float scale = 1.f) const {
#pragma unroll
    for (int e = 0; e < DPL; ++e) dst[lane_id() * DPL + e] = acc[e] * scale;
  }

  // store() with agent-scope coherent stores (dst 8-byte aligned)
  __device__ __forceinline__ void store_agent(float* dst, const float* acc) const {
    float* p = dst + lane_id() * DPL;
    if constexpr (DPL == 1) {
      st_agent(p, acc[0]);
    } else {
#pragma unroll
      for (int e = 0; e < DPL; e += 2) st_agent2(p + e, acc[e], acc[e + 1]);
    }
  }
};

// Token passes per chunk for block size B: the largest UP in {2, 1} with
// 16 * UP dividing B; 0 when B is not a multiple of 16.
// The token tile with wide V loads, for single-workgroup kernels that keep
// several tiles in flight per wave (the signed step's tail).  Q.K is that of
// TokTile.  V is loaded 16 bytes per lane: a row of D elements spans
// LPR = D / 8 lanes and one load instruction covers RPI = 64 / LPR rows, so
// a 32-token chunk of D = 128 is 8 loads instead of 32 (a wave may have at
// most 63 vector memory instructions outstanding; with one load per token
// row, two tiles in flight exceed that and the wave stalls until the first
// returns).  Lane l accumulates dims 8 (l % LPR) .. + 7 over the rows
// RPI i + l / LPR; each token's weight comes from its Q.K lane with one
// ds_bpermute per load, and the RPI lane groups are folded once, in store().
template <typename T, int NCH, int UP>
struct TokTileW : TokTile<T, NCH, UP> {
  using B = TokTile<T, NCH, UP>;
  static_assert(sizeof(T) == 2, "wide V rows take 16-bit elements");
  static constexpr int D = B::D, CH = B::CH, QW = B::QW, TPP = B::TPP, LPT = B::LPT;
  static constexpr int LPR = D / 8;              // lanes per V row
  static constexpr int RPI = STK_WAVE / LPR;     // V rows per load instruction
  static constexpr int NV = CH / RPI;            // V loads per chunk
  static constexpr int ACC = 8;                  // accumulated dims per lane
  static_assert(LPR <= STK_WAVE && CH % RPI == 0 && TPP % RPI == 0,
                "V rows must tile the chunk");

  __device__ __forceinline__ void load(const T* kb, const T* vb, int t0,
                                       uint32_t (&kw)[UP][QW], uint4 (&vw)[NV]) const {
    const T* krow = kb + (size_t)(t0 + this->slot) * D;
#pragma unroll
    for (int u = 0; u < UP; ++u) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        uint4 x = *reinterpret_cast<const uint4*>(krow + (size_t)TPP * u * D + this->kdim(c));
        kw[u][4 * c + 0] = x.x; kw[u][4 * c + 1] = x.y; kw[u][4 * c + 2] = x.z;
        kw[u][4 * c + 3] = x.w;
      }
    }
    const T* vrow = vb + (size_t)(t0 + lane_id() / LPR) * D + 8 * (lane_id() % LPR);
#pragma unroll
    for (int i = 0; i < NV; ++i) vw[i] = *reinterpret_cast<const uint4*>(vrow + (size_t)i * RPI * D);
  }

  // Online softmax over one chunk (token t0 + j valid when < Bn).  MASKV:
  // the tokens at or past Bn hold no data and their values are taken as
  // zero (a partly filled block; whatever the memory holds adds nothing).
  template <bool MASKV = false>
  __device__ __forceinline__ void update(const uint32_t* qw, const uint32_t (&kw)[UP][QW],
                                         const uint4 (&vw)[NV], int t0, int Bn, float scale,
                                         float& m, float& l, float (&acc)[ACC]) const {
    float s[UP];
    this->scores(qw, kw, t0, Bn, scale, s);
    float cm = s[0];
#pragma unroll
    for (int u = 1; u < UP; ++u) cm = fmaxf(cm, s[u]);
    cm = wave_max_u(cm);
    const float nm = fmaxf(m, cm);
    if (nm > m) {
      const float alpha = wexp(m, nm);
      l *= alpha;
#pragma unroll
      for (int e = 0; e < ACC; ++e) acc[e] *= alpha;
      m = nm;
    }
    float w[UP], ws = 0.f;
#pragma unroll
    for (int u = 0; u < UP; ++u) {
      w[u] = wexp(s[u], m);
      ws += this->part == 0 ? w[u] : 0.f;
    }
    l += wave_sum_u(ws);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int u = (RPI * i) / TPP;                       // same pass for the whole load
      const int tk = (RPI * i) % TPP + lane_id() / LPR;    // token slot within the pass
      const float wt = __shfl(w[u], tk * LPT);
      uint32_t x[4] = {vw[i].x, vw[i].y, vw[i].z, vw[i].w};
      if constexpr (MASKV) {
        const bool live = t0 + RPI * i + lane_id() / LPR < Bn;
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = live ? x[e] : 0u;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[2 * e] += wt * Elem<T>::lo(x[e]);
        acc[2 * e + 1] += wt * Elem<T>::hi(x[e]);
      }
    }
  }

  // Fold the lane groups and write D floats (times `scale`) to dst.
  __device__ __forceinline__ void store(float* dst, float (&acc)[ACC], float scale = 1.f) const {
#pragma unroll
    for (int off = LPR; off < STK_WAVE; off <<= 1)
#pragma unroll
      for (int e = 0; e < ACC; ++e) acc[e] += __shfl_xor(acc[e], off);
    if (lane_id() < LPR) {
      float4* p = reinterpret_cast<float4*>(dst + 8 * lane_id());
      p[0] = make_float4(acc[0] * scale, acc[1] * scale, acc[2] * scale, acc[3] * scale);
      p[1] = make_float4(acc[4] * scale, acc[5] * scale, acc[6] * scale, acc[7] * scale);
    }
  }
};

inline int tok_up(int b) { return b % 32 == 0 ? 2 : (b % 16 == 0 ? 1 : 0); }

// Token-tile shape for (dtype, D, B): NCH chunks per lane; 0 when unsupported.
inline int tok_nch(int dtype, int d, int b, uintptr_t align_bits) {
  if ((align_bits & 15) != 0 || tok_up(b) == 0) return 0;
  int esize = dtype == DT_F32 ? 4 : 2;
  int epc = 16 / esize;
  if (d % 64 != 0 || d % (4 * epc) != 0) return 0;
  int nch = d / (4 * epc);
  if (esize == 2 && (nch == 2 || nch == 4 || nch == 8)) return nch;
  if (esize == 4 && (nch == 4 || nch == 8)) return nch;
  return 0;
}

}  // namespace stk

// Dispatch: binds T, NCH for EXPR when the token tile supports (dtype, d).
#define STK_DISPATCH_TOK(dtype, nch, EXPR)                          \
  do {                                                              \
    if (dtype == stk::DT_BF16) {                                    \
      using T = stk::bf16s;                                         \
      if (nch == 2) { constexpr int NCH = 2; EXPR; }                \
      else if (nch == 4) { constexpr int NCH = 4; EXPR; }           \
      else { constexpr int NCH = 8; EXPR; }                         \
    } else if (dtype == stk::DT_F16) {                              \
      using T = stk::f16s;                                          \
      if (nch == 2) { constexpr int NCH = 2; EXPR; }                \
      else if (nch == 4) { constexpr int NCH = 4; EXPR; }           \
      else { constexpr int NCH = 8; EXPR; }                         \
    } else {                                                        \
      using T = float;                                              \
      if (nch == 4) { constexpr int NCH = 4; EXPR; }                \
      else { constexpr int NCH = 8; EXPR; }                         \
    }                                                               \
  } while (0)
