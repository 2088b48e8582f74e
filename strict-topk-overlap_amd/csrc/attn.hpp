// Wave-level softmax state of one (query head, KV block) pair.
//
// One 64-lane wave streams a block of B tokens x D dims.  `lpt` lanes share a
// token row (lane `part` owns NC chunks of VEC contiguous dims, chunk index
// part + c*lpt), so a wave covers tpw = 64/lpt tokens per step and U steps are
// loaded before any arithmetic to keep 16-byte loads in flight.  Scores use
// FP32 products of the converted elements, scaled by D^-1/2 after the dot
// product.  The running state (m, l, acc) follows the online softmax:
// m is wave-uniform; l and acc are per-lane partial sums over that lane's
// tokens and are combined across token lanes by wave_finish().
#pragma once

#include "common.hpp"

namespace stk {

// VEC consecutive elements of type T held as raw 32-bit words; loaded with
// one 2/4/8/16-byte access and converted to FP32 on use.
template <typename T, int VEC>
struct Raw {
  static constexpr int BYTES = VEC * (int)sizeof(T);
  static constexpr int W = BYTES >= 4 ? BYTES / 4 : 1;
  uint32_t w[W];

  __device__ __forceinline__ void load(const T* p) {
    if constexpr (BYTES == 16) {
      uint4 x = *reinterpret_cast<const uint4*>(p);
      w[0] = x.x; w[1] = x.y; w[2] = x.z; w[3] = x.w;
    } else if constexpr (BYTES == 8) {
      uint2 x = *reinterpret_cast<const uint2*>(p);
      w[0] = x.x; w[1] = x.y;
    } else if constexpr (BYTES == 4) {
      w[0] = *reinterpret_cast<const uint32_t*>(p);
    } else {
      w[0] = *reinterpret_cast<const uint16_t*>(p);
    }
  }
  __device__ __forceinline__ void zero_unless(bool keep) {
#pragma unroll
    for (int i = 0; i < W; ++i) w[i] = keep ? w[i] : 0u;
  }
  __device__ __forceinline__ float get(int i) const {
    if constexpr (sizeof(T) == 4) {
      return __uint_as_float(w[i]);
    } else {
      uint32_t bits = (w[i / 2] >> (16 * (i % 2))) & 0xffffu;
      T x;
      __builtin_memcpy(&x, &bits, 2);
      return cvt(x);
    }
  }
};

template <typename T, int VEC, int NC>
struct Tile {
  static constexpr int R = VEC * NC;   // registers per lane
  int lpt, tpw, part, tok, D;

  __device__ __forceinline__ void init(int d) {
    D = d;
    int chunks = (d + VEC - 1) / VEC;
    int per = (chunks + NC - 1) / NC;
    int l = 1;
    while (l < per) l <<= 1;
    lpt = l > STK_WAVE ? STK_WAVE : l;
    tpw = STK_WAVE / lpt;
    int lane = lane_id();
    part = lane & (lpt - 1);
    tok = lane / lpt;
  }

  __device__ __forceinline__ bool chunk_ok(int c) const { return (part + c * lpt) * VEC < D; }

  // q row -> per-lane FP32 registers (0 outside D).  Every access is issued
  // unconditionally from a clamped address so that no branch separates the
  // loads (a branch makes the compiler wait for each load in turn).
  __device__ __forceinline__ void load_q(const T* q, float* qr) const {
    Raw<T, VEC> r[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) r[c].load(q + (chunk_ok(c) ? (part + c * lpt) * VEC : 0));
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      bool ok = chunk_ok(c);
#pragma unroll
      for (int i = 0; i < VEC; ++i) qr[c * VEC + i] = ok ? r[c].get(i) : 0.f;
    }
  }

  // One token row: chunks beyond D, and rows with !valid, read a valid
  // address and are zeroed.
  __device__ __forceinline__ void load_row(const T* row, Raw<T, VEC>* dst, bool valid) const {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      bool ok = valid && chunk_ok(c);
      dst[c].load(row + (ok ? (part + c * lpt) * VEC : 0));
      dst[c].zero_unless(ok);
    }
  }

  // Raw K (and V) rows of one chunk of U * tpw tokens starting at t0.
  template <int U, bool WITH_V>
  __device__ __forceinline__ void load_chunk(const T* kb, const T* vb, int t0, int B,
                                             Raw<T, VEC> (&kr)[U][NC],
                                             Raw<T, VEC> (&vr)[U][NC]) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int t = t0 + u * tpw + tok;
      bool valid = t < B;
      load_row(kb + (size_t)(valid ? t : 0) * D, kr[u], valid);
      if constexpr (WITH_V) load_row(vb + (size_t)(valid ? t : 0) * D, vr[u], valid);
    }
  }

  // Online-softmax update of (m, l, acc) with one loaded chunk.  FIXED keeps
  // m as the exponent frame (weights exp(s - m), no rescaling).
  template <int U, bool FIXED, bool WITH_V>
  __device__ __forceinline__ void update_chunk(const float* qr, const Raw<T, VEC> (&kr)[U][NC],
                                               const Raw<T, VEC> (&vr)[U][NC], int t0, int B,
                                               float scale, float& m, float& l,
                                               float* acc) const {
    float s[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float dot = 0.f;
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int i = 0; i < VEC; ++i) dot += kr[u][c].get(i) * qr[c * VEC + i];
      for (int off = 1; off < lpt; off <<= 1) dot += __shfl_xor(dot, off);
      int t = t0 + u * tpw + tok;
      s[u] = (t < B) ? dot * scale : -INFINITY;
    }
    if constexpr (!FIXED) {
      float tile = s[0];
#pragma unroll
      for (int u = 1; u < U; ++u) tile = fmaxf(tile, s[u]);
      for (int off = lpt; off < STK_WAVE; off <<= 1) tile = fmaxf(tile, __shfl_xor(tile, off));
      float nm = fmaxf(m, tile);
      if (nm > m) {
        float alpha = (m == -INFINITY) ? 0.f : expf(m - nm);
        l *= alpha;
#pragma unroll
        for (int i = 0; i < R; ++i) acc[i] *= alpha;
        m = nm;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float w = (s[u] == -INFINITY) ? 0.f : expf(s[u] - m);
      l += w;
      if constexpr (WITH_V) {
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[c * VEC + i] += w * vr[u][c].get(i);
      }
    }
  }

  // Accumulate one block into (m, l, acc).  WITH_V=false skips V.
  template <int U, bool FIXED, bool WITH_V>
  __device__ __forceinline__ void accum(const float* qr, const T* kb, const T* vb, int B,
                                        float scale, float& m, float& l, float* acc) const {
    for (int t0 = 0; t0 < B; t0 += U * tpw) {
      Raw<T, VEC> kr[U][NC];
      Raw<T, VEC> vr[U][NC];
      load_chunk<U, WITH_V>(kb, vb, t0, B, kr, vr);
      update_chunk<U, FIXED, WITH_V>(qr, kr, vr, t0, B, scale, m, l, acc);
    }
  }

  // Same as accum but also returns, per lane, sum |w * v| (compact low walk).
  template <int U>
  __device__ __forceinline__ void accum_fixed_abs(const float* qr, const T* kb, const T* vb, int B,
                                                  float scale, float m, float& l, float* acc,
                                                  float* abs_acc) const {
    for (int t0 = 0; t0 < B; t0 += U * tpw) {
      Raw<T, VEC> kr[U][NC];
      Raw<T, VEC> vr[U][NC];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int t = t0 + u * tpw + tok;
        bool valid = t < B;
        load_row(kb + (size_t)(valid ? t : 0) * D, kr[u], valid);
        load_row(vb + (size_t)(valid ? t : 0) * D, vr[u], valid);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float dot = 0.f;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int i = 0; i < VEC; ++i) dot += kr[u][c].get(i) * qr[c * VEC + i];
        for (int off = 1; off < lpt; off <<= 1) dot += __shfl_xor(dot, off);
        int t = t0 + u * tpw + tok;
        float w = (t < B) ? expf(dot * scale - m) : 0.f;
        l += w;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            float x = w * vr[u][c].get(i);
            acc[c * VEC + i] += x;
            abs_acc[c * VEC + i] += fabsf(x);
          }
      }
    }
  }

  // Combine per-lane partial sums across the token lanes of the wave.
  __device__ __forceinline__ void finish(float& l, float* acc) const {
    for (int off = lpt; off < STK_WAVE; off <<= 1) {
      l += __shfl_xor(l, off);
#pragma unroll
      for (int i = 0; i < R; ++i) acc[i] += __shfl_xor(acc[i], off);
    }
  }

  // Lanes with tok == 0 write the D-vector (optionally scaled).
  __device__ __forceinline__ void store(float* dst, const float* acc, float scale = 1.f) const {
    if (tok != 0) return;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      int base = (part + c * lpt) * VEC;
      if (VEC > 1) {
        if (base < D) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) dst[base + i] = acc[c * VEC + i] * scale;
        }
      } else {
        if (base < D) dst[base] = acc[c] * scale;
      }
    }
  }
};

// Configuration choice shared by every launcher: vector tiles when D is a
// multiple of the 16-byte vector and fits one wave, scalar tiles otherwise.
template <typename T>
struct VecOf { static constexpr int value = 16 / sizeof(T); };

inline bool use_vec(int dtype, int d) {
  int vec = dtype == DT_F32 ? 4 : 8;
  return d % vec == 0 && d / vec <= STK_WAVE;
}

constexpr int kMaxD = 1024;   // scalar tiles: NC = 16 chunks of 1 per lane

}  // namespace stk

// Dispatch macro: binds T, VEC, NC, U for the kernel launch expression EXPR.
#define STK_DISPATCH_TILE(dtype, d, EXPR)                                    \
  do {                                                                       \
    bool _vec = stk::use_vec(dtype, d);                                      \
    if (dtype == stk::DT_BF16) {                                             \
      using T = stk::bf16s;                                                  \
      if (_vec) { constexpr int VEC = 8, NC = 1, U = 8; EXPR; }              \
      else { constexpr int VEC = 1, NC = 16, U = 1; EXPR; }                  \
    } else if (dtype == stk::DT_F16) {                                       \
      using T = stk::f16s;                                                   \
      if (_vec) { constexpr int VEC = 8, NC = 1, U = 8; EXPR; }              \
      else { constexpr int VEC = 1, NC = 16, U = 1; EXPR; }                  \
    } else {                                                                 \
      using T = float;                                                       \
      if (_vec) { constexpr int VEC = 4, NC = 1, U = 8; EXPR; }              \
      else { constexpr int VEC = 1, NC = 16, U = 1; EXPR; }                  \
    }                                                                        \
  } while (0)
