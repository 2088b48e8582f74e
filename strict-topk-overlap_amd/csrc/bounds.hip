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
// k_bounds: one workgroup per (KV head, block).  Thread (g, c) reads 16-byte
// chunks c of token rows g, g + TG, ... (TG = 256 / (D / EPC) token groups),
// so each wave instruction reads whole rows; the TG partial min/max are folded
// through LDS.  HBM-bound: B * D * e bytes read and 8 * D bytes written per
// block.
#include "common.hpp"
#include "api.hpp"

namespace stk {

struct BoundsArgs {
  const void* k; int dtype;
  int rows;          // hkv * n blocks
  int b, d;
  float* lo; float* hi;
};

// NaN-propagating min / max (torch.amin / amax semantics)
__device__ __forceinline__ float nmin(float m, float v) { return (v < m || v != v) ? v : m; }
__device__ __forceinline__ float nmax(float m, float v) { return (v > m || v != v) ? v : m; }

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
    a.lo[(size_t)row * a.d + x] = l;
    a.hi[(size_t)row * a.d + x] = h;
  }
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
    a.lo[(size_t)row * a.d + x] = l;
    a.hi[(size_t)row * a.d + x] = h;
  }
}

struct AppendArgs {
  const void* k; int dtype;   // new token's keys [hkv, d]
  int hkv, n, d, block, pos;
  float* lo; float* hi;
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
  a.lo[o] = a.pos == 0 ? v : nmin(a.lo[o], v);
  a.hi[o] = a.pos == 0 ? v : nmax(a.hi[o], v);
}

}  // namespace stk

using namespace stk;

extern "C" {

STK_API int stk_block_bounds(const void* k, int dtype, int hkv, int n, int b, int d, float* lo,
                             float* hi, void* stream) {
  STK_REQUIRE(k && lo && hi, "null pointer");
  STK_REQUIRE(dtype == DT_F32 || dtype == DT_F16 || dtype == DT_BF16, "unsupported dtype");
  STK_REQUIRE(hkv > 0 && n >= 0 && b > 0 && d > 0, "bad shape");
  if (n == 0) return STK_OK;
  STK_REQUIRE((int64_t)hkv * n <= 0x7fffffff, "too many blocks");
  BoundsArgs a{k, dtype, hkv * n, b, d, lo, hi};
  hipStream_t st = (hipStream_t)stream;
  const bool vec = dtype != DT_F32 && d % 8 == 0 && d <= 2048 &&
                   (reinterpret_cast<uintptr_t>(k) & 15) == 0;
  if (vec && dtype == DT_BF16)
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
                              int pos, float* lo, float* hi, void* stream) {
  STK_REQUIRE(k_new && lo && hi, "null pointer");
  STK_REQUIRE(dtype == DT_F32 || dtype == DT_F16 || dtype == DT_BF16, "unsupported dtype");
  STK_REQUIRE(hkv > 0 && n > 0 && d > 0, "bad shape");
  STK_REQUIRE(block >= 0 && block < n && pos >= 0, "block or position out of range");
  AppendArgs a{k_new, dtype, hkv, n, d, block, pos, lo, hi};
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

}  // extern "C"
