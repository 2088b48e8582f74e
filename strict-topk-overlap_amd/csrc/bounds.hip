// Block metadata for the bound scorer: per-block, per-dim key minimum and
// maximum (lo, hi), built at prefill and updated on every decode append.
//
// Reference: the harness builds them outside the timed step as
// k.amin(dim=2).float(), k.amax(dim=2).float()
// (benchmarks/critical_path.py:186, benchmarks/run_benchmark.py:43,
// tests/check_gqa.py:47); a decode loop needs the same per-token update when
// a token is appended to the last block.  Like torch.amin / amax, a NaN key
// makes the bound NaN.
//
// k_bounds_cols (16-bit keys, 16-byte aligned rows): one thread per (block,
// 16-byte column); k_bounds (unaligned lo/hi): one workgroup per block, token
// groups folded through LDS; k_bounds_any: every other case.  HBM-bound:
// B * D * e bytes read and 8 * D bytes written per block (4 * D with lb:
// the bounds stored in the keys' own 16-bit type, exact since they are
// values of that type).
#include "common.hpp"
#include "api.hpp"

namespace stk {

struct BoundsArgs {
  const void* k; int dtype;
  int rows;          // hkv * n blocks
  int b, d;
  void* lo; void* hi;
  int lb;            // 1: lo / hi in T (16-bit), else FP32
};

// NaN-propagating min / max (torch.amin / amax semantics)
__device__ __forceinline__ float nmin(float m, float v) { return (v < m || v != v) ? v : m; }
__device__ __forceinline__ float nmax(float m, float v) { return (v > m || v != v) ? v : m; }

// FP32 -> T bits for a value that is exactly a T value (a bound is one of
// the keys), NaN payload kept.
template <typename T> __device__ __forceinline__ uint16_t bits16(float v);
template <> __device__ __forceinline__ uint16_t bits16<bf16s>(float v) {
  return (uint16_t)(__float_as_uint(v) >> 16);
}
template <> __device__ __forceinline__ uint16_t bits16<f16s>(float v) {
  const _Float16 h = (_Float16)v;
  uint16_t r;
  __builtin_memcpy(&r, &h, 2);
  return r;
}
template <> __device__ __forceinline__ uint16_t bits16<float>(float) { return 0; }

// Bound element i of p, stored as FP32 or (lb) as T.
template <typename T>
__device__ __forceinline__ float get_bound(const void* p, size_t i, bool lb) {
  if constexpr (sizeof(T) == 2)
    if (lb) return cvt(T{static_cast<const uint16_t*>(p)[i]});
  return static_cast<const float*>(p)[i];
}
template <typename T>
__device__ __forceinline__ void put_bound(void* p, size_t i, float v, bool lb) {
  if constexpr (sizeof(T) == 2)
    if (lb) {
      static_cast<uint16_t*>(p)[i] = bits16<T>(v);
      return;
    }
  static_cast<float*>(p)[i] = v;
}

template <typename T>
__device__ __forceinline__ void unpack8(const uint4& x, float (&f)[8]) {
  if constexpr (sizeof(T) == 2) {
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = cvt(T{uint16_t(w[i] & 0xffffu)});
      f[2 * i + 1] = cvt(T{uint16_t(w[i] >> 16)});
    }
  }
}

// Vector path: 16-bit elements, D % 8 == 0, D <= 2048, 16-byte aligned rows.
template <typename T>
__global__ __launch_bounds__(256) void k_bounds(BoundsArgs a) {
  __shared__ float s_lo[256 * 8], s_hi[256 * 8];
  const int row = blockIdx.x;
  const int cpr = a.d / 8;                 // 16-byte chunks per token row
  const int tg = blockDim.x / cpr;         // token groups
  const int c = threadIdx.x % cpr, g = threadIdx.x / cpr;
  float lo[8], hi[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    lo[e] = INFINITY;
    hi[e] = -INFINITY;
  }
  const T* base = reinterpret_cast<const T*>(a.k) + (size_t)row * a.b * a.d + 8 * c;
  if (g < tg) {
    for (int t = g; t < a.b; t += tg) {
      float f[8];
      unpack8<T>(*reinterpret_cast<const uint4*>(base + (size_t)t * a.d), f);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        lo[e] = nmin(lo[e], f[e]);
        hi[e] = nmax(hi[e], f[e]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    s_lo[e * 256 + threadIdx.x] = lo[e];
    s_hi[e * 256 + threadIdx.x] = hi[e];
  }
  __syncthreads();
  for (int x = threadIdx.x; x < a.d; x += blockDim.x) {
    const int cc = x / 8, e = x % 8;
    float l = INFINITY, h = -INFINITY;
    for (int gg = 0; gg < tg; ++gg) {
      l = nmin(l, s_lo[e * 256 + gg * cpr + cc]);
      h = nmax(h, s_hi[e * 256 + gg * cpr + cc]);
    }
    put_bound<T>(a.lo, (size_t)row * a.d + x, l, a.lb);
    put_bound<T>(a.hi, (size_t)row * a.d + x, h, a.lb);
  }
}

// Column path: one thread per (block, 16-byte column of D).  The thread
// streams its column down the block's B token rows, 16 loads of 16 bytes in
// flight, and writes its 8 dims of lo and hi with two 16-byte stores each: no
// LDS and no barrier.  One wave instruction reads 256-byte row segments of
// 64 / (D / 8) consecutive blocks.  (Measured on c3's K, 151 MB: 30 us; the
// one-block-per-workgroup layout below folds its token groups through LDS
// with 8-way bank conflicts, 37 us.)
#ifndef STK_BOUNDS_WG
#define STK_BOUNDS_WG 64
#endif
#ifndef STK_BOUNDS_UNR
#define STK_BOUNDS_UNR 16
#endif
template <typename T>
__global__ __launch_bounds__(STK_BOUNDS_WG) void k_bounds_cols(BoundsArgs a) {
  const int cpr = a.d / 8;
  const int64_t gt = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gt >= (int64_t)a.rows * cpr) return;
  const int row = (int)(gt / cpr), c = (int)(gt % cpr);
  const T* base = reinterpret_cast<const T*>(a.k) + (size_t)row * a.b * a.d + 8 * c;
  float lo[8], hi[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    lo[e] = INFINITY;
    hi[e] = -INFINITY;
  }
  constexpr int U = STK_BOUNDS_UNR;
  for (int t0 = 0; t0 < a.b; t0 += U) {
    uint4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + u < a.b ? t0 + u : t0;   // past B: token t0 again
      x[u] = *reinterpret_cast<const uint4*>(base + (size_t)t * a.d);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float f[8];
      unpack8<T>(x[u], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        lo[e] = nmin(lo[e], f[e]);
        hi[e] = nmax(hi[e], f[e]);
      }
    }
  }
  const size_t o = (size_t)row * a.d + 8 * c;
  if (a.lb) {
    uint32_t wl[4], wh[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wl[i] = bits16<T>(lo[2 * i]) | ((uint32_t)bits16<T>(lo[2 * i + 1]) << 16);
      wh[i] = bits16<T>(hi[2 * i]) | ((uint32_t)bits16<T>(hi[2 * i + 1]) << 16);
    }
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.lo) + o) =
        make_uint4(wl[0], wl[1], wl[2], wl[3]);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.hi) + o) =
        make_uint4(wh[0], wh[1], wh[2], wh[3]);
    return;
  }
  float4* ol = reinterpret_cast<float4*>(static_cast<float*>(a.lo) + o);
  float4* oh = reinterpret_cast<float4*>(static_cast<float*>(a.hi) + o);
  ol[0] = make_float4(lo[0], lo[1], lo[2], lo[3]);
  ol[1] = make_float4(lo[4], lo[5], lo[6], lo[7]);
  oh[0] = make_float4(hi[0], hi[1], hi[2], hi[3]);
  oh[1] = make_float4(hi[4], hi[5], hi[6], hi[7]);
}

// Generic path: any element type and D; thread per (block, dim).
template <typename T>
__global__ __launch_bounds__(256) void k_bounds_any(BoundsArgs a) {
  const int row = blockIdx.x;
  const T* base = reinterpret_cast<const T*>(a.k) + (size_t)row * a.b * a.d;
  for (int x = threadIdx.x; x < a.d; x += blockDim.x) {
    float l = INFINITY, h = -INFINITY;
    for (int t = 0; t < a.b; ++t) {
      const float v = cvt(base[(size_t)t * a.d + x]);
      l = nmin(l, v);
      h = nmax(h, v);
    }
    put_bound<T>(a.lo, (size_t)row * a.d + x, l, a.lb);
    put_bound<T>(a.hi, (size_t)row * a.d + x, h, a.lb);
  }
}

struct AppendArgs {
  const void* k; int dtype;   // new token's keys [hkv, d]
  int hkv, n, d, block, pos;
  void* lo; void* hi; int lb;
};

// One appended token: block `block` of every KV head starts over at pos 0,
// otherwise widens its bounds.
template <typename T>
__global__ __launch_bounds__(256) void k_bounds_append(AppendArgs a) {
  const int x = blockIdx.x * blockDim.x + threadIdx.x;
  if (x >= a.hkv * a.d) return;
  const int kv = x / a.d, dim = x % a.d;
  const float v = cvt(reinterpret_cast<const T*>(a.k)[x]);
  const size_t o = ((size_t)kv * a.n + a.block) * a.d + dim;
  put_bound<T>(a.lo, o, a.pos == 0 ? v : nmin(get_bound<T>(a.lo, o, a.lb), v), a.lb);
  put_bound<T>(a.hi, o, a.pos == 0 ? v : nmax(get_bound<T>(a.hi, o, a.lb), v), a.lb);
}

// One decode token per request into a paged pool (the paged wire format of
// paged.hip): thread (r, kvh, dim) writes K/V element dim of KV head kvh at
// token position positions[r] (block pos / B, offset pos % B) into that
// block's page, widens the page's lo/hi by it (offset 0 starts them over),
// and one thread per request sets nblocks[r] = pos / B + 1 and (when given)
// ntokens[r] = pos + 1, after checking that the block has a valid page for
// every KV head.  A position outside [0, nb * B) writes nothing; a block on an
// invalid page writes nothing for that KV head and leaves the counts as
// they were.
struct PagedAppendArgs {
  const void* k_new; const void* v_new;   // [R, Hkv, D]
  int requests, hkv, nb, b, d, pages;
  void* k_pages; void* v_pages;           // [P, B, D]
  void* lo; void* hi;                     // [P, D], FP32 or (lb) T
  int lb;
  const int32_t* table;                   // [R, Hkv, nb]
  int32_t* nblocks;                       // [R]
  int32_t* ntokens;                       // [R] or null
  const int32_t* positions;               // [R]
};

template <typename T>
__global__ __launch_bounds__(256) void k_paged_append(PagedAppendArgs a) {
  const int64_t x = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (x >= (int64_t)a.requests * a.hkv * a.d) return;
  const int dim = (int)(x % a.d);
  const int rk = (int)(x / a.d);              // r * hkv + kvh
  const int r = rk / a.hkv;
  const int pos = a.positions[r];
  if (pos < 0 || pos >= a.nb * a.b) return;
  const int blk = pos / a.b, off = pos % a.b;
  if (rk % a.hkv == 0 && dim == 0) {
    bool ok = true;
    for (int kh = 0; kh < a.hkv; ++kh) {
      const int pk = a.table[((int64_t)rk + kh) * a.nb + blk];
      ok = ok && pk >= 0 && pk < a.pages;
    }
    if (ok) {
      a.nblocks[r] = blk + 1;
      if (a.ntokens) a.ntokens[r] = pos + 1;
    }
  }
  const int page = a.table[(int64_t)rk * a.nb + blk];
  if (page < 0 || page >= a.pages) return;
  const T kv = reinterpret_cast<const T*>(a.k_new)[x];
  const size_t o = ((size_t)page * a.b + off) * a.d + dim;
  reinterpret_cast<T*>(a.k_pages)[o] = kv;
  reinterpret_cast<T*>(a.v_pages)[o] = reinterpret_cast<const T*>(a.v_new)[x];
  const float f = cvt(kv);
  const size_t ob = (size_t)page * a.d + dim;
  put_bound<T>(a.lo, ob, off == 0 ? f : nmin(get_bound<T>(a.lo, ob, a.lb), f), a.lb);
  put_bound<T>(a.hi, ob, off == 0 ? f : nmax(get_bound<T>(a.hi, ob, a.lb), f), a.lb);
}

}  // namespace stk

using namespace stk;

extern "C" {

STK_API int stk_block_bounds(const void* k, int dtype, int hkv, int n, int b, int d, void* lo,
                             void* hi, int bounds_dtype, void* stream) {
  STK_REQUIRE(k && lo && hi, "null pointer");
  STK_REQUIRE(dtype == DT_F32 || dtype == DT_F16 || dtype == DT_BF16, "unsupported dtype");
  STK_REQUIRE(stk_bounds_ok(dtype, bounds_dtype), "lo and hi must be FP32 or K's 16-bit type");
  STK_REQUIRE(hkv > 0 && n >= 0 && b > 0 && d > 0, "bad shape");
  if (n == 0) return STK_OK;
  STK_REQUIRE((int64_t)hkv * n <= 0x7fffffff, "too many blocks");
  BoundsArgs a{k, dtype, hkv * n, b, d, lo, hi, bounds_dtype != 0};
  hipStream_t st = (hipStream_t)stream;
  const bool vec = dtype != DT_F32 && d % 8 == 0 && d <= 2048 &&
                   (reinterpret_cast<uintptr_t>(k) & 15) == 0;
  // the column path needs 16-byte aligned lo/hi rows as well
  const bool vec16 = vec && ((reinterpret_cast<uintptr_t>(lo) | reinterpret_cast<uintptr_t>(hi)) &
                             15) == 0;
  const int64_t threads = (int64_t)a.rows * (d / 8);
  const bool cols = vec16 && (threads + STK_BOUNDS_WG - 1) / STK_BOUNDS_WG <= 0x7fffffff;
  const dim3 cgrid((unsigned)((threads + STK_BOUNDS_WG - 1) / STK_BOUNDS_WG));
  if (cols && dtype == DT_BF16) {
    hipLaunchKernelGGL(k_bounds_cols<bf16s>, cgrid, dim3(STK_BOUNDS_WG), 0, st, a);
  } else if (cols) {
    hipLaunchKernelGGL(k_bounds_cols<f16s>, cgrid, dim3(STK_BOUNDS_WG), 0, st, a);
  } else if (vec && dtype == DT_BF16)
    hipLaunchKernelGGL(k_bounds<bf16s>, dim3(a.rows), dim3(256), 0, st, a);
  else if (vec)
    hipLaunchKernelGGL(k_bounds<f16s>, dim3(a.rows), dim3(256), 0, st, a);
  else if (dtype == DT_BF16)
    hipLaunchKernelGGL(k_bounds_any<bf16s>, dim3(a.rows), dim3(256), 0, st, a);
  else if (dtype == DT_F16)
    hipLaunchKernelGGL(k_bounds_any<f16s>, dim3(a.rows), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(k_bounds_any<float>, dim3(a.rows), dim3(256), 0, st, a);
  return stk_check_launch("k_bounds");
}

STK_API int stk_bounds_append(const void* k_new, int dtype, int hkv, int n, int d, int block,
                              int pos, void* lo, void* hi, int bounds_dtype, void* stream) {
  STK_REQUIRE(k_new && lo && hi, "null pointer");
  STK_REQUIRE(dtype == DT_F32 || dtype == DT_F16 || dtype == DT_BF16, "unsupported dtype");
  STK_REQUIRE(stk_bounds_ok(dtype, bounds_dtype), "lo and hi must be FP32 or K's 16-bit type");
  STK_REQUIRE(hkv > 0 && n > 0 && d > 0, "bad shape");
  STK_REQUIRE(block >= 0 && block < n && pos >= 0, "block or position out of range");
  AppendArgs a{k_new, dtype, hkv, n, d, block, pos, lo, hi, bounds_dtype != 0};
  const int grid = (hkv * d + 255) / 256;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DT_BF16)
    hipLaunchKernelGGL(k_bounds_append<bf16s>, dim3(grid), dim3(256), 0, st, a);
  else if (dtype == DT_F16)
    hipLaunchKernelGGL(k_bounds_append<f16s>, dim3(grid), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(k_bounds_append<float>, dim3(grid), dim3(256), 0, st, a);
  return stk_check_launch("k_bounds_append");
}

STK_API int stk_paged_append(const void* k_new, const void* v_new, int dtype, int requests,
                             int hkv, int nb, int b, int d, int pages, void* k_pages,
                             void* v_pages, void* lo_pages, void* hi_pages, int bounds_dtype,
                             const int32_t* block_table, int32_t* nblocks, int32_t* ntokens,
                             const int32_t* positions, void* stream) {
  STK_REQUIRE(k_new && v_new && k_pages && v_pages && lo_pages && hi_pages && block_table &&
                  nblocks && positions,
              "null pointer");
  STK_REQUIRE(dtype == DT_F32 || dtype == DT_F16 || dtype == DT_BF16, "unsupported dtype");
  STK_REQUIRE(requests > 0 && hkv > 0 && nb > 0 && b > 0 && d > 0 && pages > 0, "bad shape");
  STK_REQUIRE(stk_bounds_ok(dtype, bounds_dtype),
              "lo and hi pages must be FP32 or the pages' 16-bit type");
  STK_REQUIRE((int64_t)nb * b <= 0x7fffffff && (int64_t)requests * hkv * d <= 0x7fffffff,
              "shape too large");
  PagedAppendArgs a{k_new, v_new, requests, hkv, nb, b, d, pages, k_pages, v_pages, lo_pages,
                    hi_pages, bounds_dtype != 0, block_table, nblocks, ntokens, positions};
  const int64_t n = (int64_t)requests * hkv * d;
  const dim3 grid((unsigned)((n + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DT_BF16)
    hipLaunchKernelGGL(k_paged_append<bf16s>, grid, dim3(256), 0, st, a);
  else if (dtype == DT_F16)
    hipLaunchKernelGGL(k_paged_append<f16s>, grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(k_paged_append<float>, grid, dim3(256), 0, st, a);
  return stk_check_launch("k_paged_append");
}

}  // extern "C"
