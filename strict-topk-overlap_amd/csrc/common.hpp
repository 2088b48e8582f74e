// Shared device helpers for the gfx950 strict-topk kernels.
//
// Element types are carried as raw 16/32-bit storage and converted to FP32
// in registers.  All kernels are written for 64-wide wavefronts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#define STK_WAVE 64

namespace stk {

enum DType : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };
enum IType : int { IT_I32 = 0, IT_I64 = 1 };

struct bf16s { uint16_t x; };
struct f16s { uint16_t x; };

__device__ __forceinline__ float cvt(float x) { return x; }
__device__ __forceinline__ float cvt(bf16s x) { return __uint_as_float(uint32_t(x.x) << 16); }
__device__ __forceinline__ float cvt(f16s x) {
  _Float16 h;
  __builtin_memcpy(&h, &x.x, 2);
  return (float)h;
}

// Unpack one 32-bit word holding 2 (16-bit types) or 1 (fp32) elements.
template <typename T> struct Unpack;
template <> struct Unpack<float> {
  static constexpr int per_word = 1;
  __device__ __forceinline__ static void run(uint32_t w, float* out) { out[0] = __uint_as_float(w); }
};
template <> struct Unpack<bf16s> {
  static constexpr int per_word = 2;
  __device__ __forceinline__ static void run(uint32_t w, float* out) {
    out[0] = __uint_as_float(w << 16);
    out[1] = __uint_as_float(w & 0xffff0000u);
  }
};
template <> struct Unpack<f16s> {
  static constexpr int per_word = 2;
  __device__ __forceinline__ static void run(uint32_t w, float* out) {
    f16s a{uint16_t(w & 0xffffu)}, b{uint16_t(w >> 16)};
    out[0] = cvt(a);
    out[1] = cvt(b);
  }
};

// Load VEC contiguous elements starting at p (aligned to VEC*sizeof(T) when
// that is 4, 8 or 16 bytes) and convert to FP32.
template <typename T, int VEC>
__device__ __forceinline__ void load_vec(const T* p, float* out) {
  constexpr int bytes = VEC * (int)sizeof(T);
  if constexpr (bytes == 16) {
    uint4 w = *reinterpret_cast<const uint4*>(p);
    constexpr int pw = Unpack<T>::per_word;
    Unpack<T>::run(w.x, out + 0 * pw);
    Unpack<T>::run(w.y, out + 1 * pw);
    Unpack<T>::run(w.z, out + 2 * pw);
    Unpack<T>::run(w.w, out + 3 * pw);
  } else if constexpr (bytes == 8) {
    uint2 w = *reinterpret_cast<const uint2*>(p);
    constexpr int pw = Unpack<T>::per_word;
    Unpack<T>::run(w.x, out);
    Unpack<T>::run(w.y, out + pw);
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) out[i] = cvt(p[i]);
  }
}

__device__ __forceinline__ int64_t load_id(const void* ids, int itype, int64_t i) {
  return itype == IT_I64 ? reinterpret_cast<const int64_t*>(ids)[i]
                         : (int64_t)reinterpret_cast<const int32_t*>(ids)[i];
}
__device__ __forceinline__ void store_id(void* ids, int itype, int64_t i, int64_t v) {
  if (itype == IT_I64) reinterpret_cast<int64_t*>(ids)[i] = v;
  else reinterpret_cast<int32_t*>(ids)[i] = (int32_t)v;
}

// Q, K, V of one call: q[hq, d]; k, v[hkv, n, b, d]; head h reads KV head h / (hq / hkv).
struct KV {
  const void* q; const void* k; const void* v;
  int hq, hkv, n, b, d;
};

// Branch-free guarded load: the access is always issued (from index 0 when
// !ok, which callers guarantee to be valid), and the value replaced after.
// Keeping loads out of branches lets the compiler keep them all in flight.
template <typename X>
__device__ __forceinline__ X ld_or(const X* p, int64_t i, bool ok, X other) {
  X v = p[ok ? i : 0];
  return ok ? v : other;
}

// Paged, batched KV.  A batch of requests is flattened into hq = R * Hq query
// heads and hkv = R * Hkv KV rows (KV row r * Hkv + kvh: KV head kvh of
// request r).  K/V live in pages [P, B, D] (one page = one KV head's block of
// B tokens) and the block bounds in lo/hi pages [P, D];
// table[kv * n + j] is the page of logical block j of KV row kv (n = the
// table's row width), valid for j < nblk[kv / hkv_req].  A table entry
// outside [0, pages) is an invalid page: its block has the empty state and
// scores lowest, and nothing is read from it.  ntok (optional) holds each
// request's token count: token t of block j holds data when j * B + t <
// ntok[r], so a request's last block may be partly filled (the tokens past
// the count are never weighted, whatever the page holds there); without it
// every block holds B tokens.
//
// btable (optional) gives the scorer its own table into the lo/hi pages, of
// bpages rows: with a host-backed cache, K/V pages are resident for only
// some blocks (table holds -1 for the others, whose blocks then have the
// empty state), while every block's bounds stay on the device and every
// block is scored.  Without btable the scorer uses table.
struct Paging {
  const int32_t* table;
  const int32_t* nblk;
  int hkv_req;
  int pages;
  const int32_t* ntok;
  const int32_t* btable;
  int bpages;
};

// Bounds row of block j of KV row kv when ok, else -1 (the load always
// issued, as in pg_page).
__device__ __forceinline__ int pg_bounds_row(const Paging& pg, int kv, int n, int64_t j,
                                             bool ok) {
  const int32_t* t = pg.btable ? pg.btable : pg.table;
  const int lim = pg.btable ? pg.bpages : pg.pages;
  const int p = ld_or(t, (int64_t)kv * n + j, ok, -1);
  return (p >= 0 && p < lim) ? p : -1;
}

// Valid blocks of KV row kv, clamped to [0, n].
__device__ __forceinline__ int pg_blocks(const Paging& pg, int kv, int n) {
  const int x = pg.nblk[kv / pg.hkv_req];
  return x < 0 ? 0 : (x > n ? n : x);
}

// Token count of KV row kv's request (INT32_MAX without ntok: every block
// full); one load, meant to be issued beside the row's other entry loads.
__device__ __forceinline__ int pg_row_tokens(const Paging& pg, int kv) {
  return pg.ntok ? pg.ntok[kv / pg.hkv_req] : 0x7fffffff;
}

// Tokens of block j holding data, in [0, b], given the row's token count.
__device__ __forceinline__ int pg_block_tokens(int row_tokens, int64_t j, int b) {
  const int64_t x = (int64_t)row_tokens - j * b;
  return x <= 0 ? 0 : (x >= b ? b : (int)x);
}

// Page of block j of KV row kv when ok, else -1; the table load is always
// issued (entry 0 when !ok) so that it never sits under a branch.
__device__ __forceinline__ int pg_page(const Paging& pg, int kv, int n, int64_t j, bool ok) {
  const int p = ld_or(pg.table, (int64_t)kv * n + j, ok, -1);
  return (p >= 0 && p < pg.pages) ? p : -1;
}

template <typename I>
__device__ __forceinline__ int64_t ld_id(const void* ids, int64_t i) {
  return (int64_t) reinterpret_cast<const I*>(ids)[i];
}

// ------------------------------------------------------ DPP lane exchange
// Cross-lane moves through the VALU's data-parallel-primitive modifier
// (no LDS round trip).  Controls (GFX9 encoding): quad_perm [1,0,3,2] =
// 0xB1 (xor 1), [2,3,0,1] = 0x4E (xor 2), row_ror:r = 0x120 + r (rotate
// inside each 16-lane row), row_half_mirror = 0x141 (within 8 lanes,
// i <-> 7-i), row_mirror = 0x140 (within 16 lanes, i <-> 15-i),
// row_bcast15 = 0x142, row_bcast31 = 0x143.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                               __builtin_bit_cast(int, v), CTRL,
                                                               ROW_MASK, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
  uint64_t b = (uint64_t)__double_as_longlong(v);
  int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xf, 0xf, false);
  int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xf, 0xf, false);
  return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}

// Sum over the 4 lanes of a quad, result in all 4 lanes.
__device__ __forceinline__ float quad_sum(float v) {
  v += dpp<0xB1>(0.f, v);
  v += dpp<0x4E>(0.f, v);
  return v;
}

// Maximum over the whole wave, returned wave-uniform.  (Quads, half rows and
// rows by permutation; rows 1 and 3, then 2 and 3, by row broadcast; lane 63
// ends with the total.)
__device__ __forceinline__ float wave_max_u(float v) {
  v = fmaxf(v, dpp<0xB1>(v, v));
  v = fmaxf(v, dpp<0x4E>(v, v));
  v = fmaxf(v, dpp<0x141>(v, v));
  v = fmaxf(v, dpp<0x140>(v, v));
  v = fmaxf(v, dpp<0x142, 0xa>(v, v));
  v = fmaxf(v, dpp<0x143, 0xc>(v, v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Sum over the whole wave, returned wave-uniform (same pattern).
__device__ __forceinline__ float wave_sum_u(float v) {
  v += dpp<0xB1>(0.f, v);
  v += dpp<0x4E>(0.f, v);
  v += dpp<0x141>(0.f, v);
  v += dpp<0x140>(0.f, v);
  v += dpp<0x142, 0xa>(0.f, v);
  v += dpp<0x143, 0xc>(0.f, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// ---------------------------------------------------------------- wave ops
__device__ __forceinline__ int lane_id() { return threadIdx.x & (STK_WAVE - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / STK_WAVE; }

// Map a launch-order workgroup index to a logical index so that every XCD
// (workgroups are dealt round-robin over 8 XCDs) receives one contiguous
// range of logical workgroups.  Consecutive logical items share KV heads, so
// their tiles meet in the same XCD-local L2.  A bijection on [0, total).
__device__ __forceinline__ int xcd_remap(int w, int total) {
  constexpr int X = 8;
  int xcd = w % X, r = w / X;
  int base = total / X, extra = total % X;
  int start = xcd * base + (xcd < extra ? xcd : extra);
  return start + r;
}

template <typename F>
__device__ __forceinline__ float xor_reduce(float v, int from, int to, F op) {
  // combine lanes with xor offsets from, 2*from, ..., to (inclusive)
  for (int off = from; off <= to; off <<= 1) v = op(v, __shfl_xor(v, off));
  return v;
}
struct OpAdd { __device__ float operator()(float a, float b) const { return a + b; } };
struct OpMax { __device__ float operator()(float a, float b) const { return fmaxf(a, b); } };

__device__ __forceinline__ float wave_sum(float v) { return xor_reduce(v, 1, 32, OpAdd()); }
__device__ __forceinline__ float wave_max(float v) { return xor_reduce(v, 1, 32, OpMax()); }

__device__ __forceinline__ int wave_any(bool p) { return __any(p); }

// Keeps N loaded values live at one point (groups of eight), so that the
// compiler moves none of their loads under a later branch and waits for them
// once.
template <int N>
__device__ __forceinline__ void hold_all(float (&x)[N]) {
  static_assert(N % 8 == 0, "groups of eight");
#pragma unroll
  for (int i = 0; i < N; i += 8)
    asm volatile("" : "+v"(x[i]), "+v"(x[i + 1]), "+v"(x[i + 2]), "+v"(x[i + 3]),
                 "+v"(x[i + 4]), "+v"(x[i + 5]), "+v"(x[i + 6]), "+v"(x[i + 7]));
}

// Wave-wide max (MAX) or min of an unsigned word, returned in every lane.
template <bool MAX>
__device__ __forceinline__ uint32_t wave_ext_u32(uint32_t v) {
  const int id = MAX ? 0 : -1;
  auto f = [&](uint32_t x, int y) {
    return MAX ? (x > (uint32_t)y ? x : (uint32_t)y) : (x < (uint32_t)y ? x : (uint32_t)y);
  };
  v = f(v, __builtin_amdgcn_update_dpp(id, (int)v, 0xB1, 0xf, 0xf, false));
  v = f(v, __builtin_amdgcn_update_dpp(id, (int)v, 0x4E, 0xf, 0xf, false));
  v = f(v, __builtin_amdgcn_update_dpp(id, (int)v, 0x141, 0xf, 0xf, false));
  v = f(v, __builtin_amdgcn_update_dpp(id, (int)v, 0x140, 0xf, 0xf, false));
  v = f(v, __builtin_amdgcn_update_dpp(id, (int)v, 0x142, 0xa, 0xf, false));
  v = f(v, __builtin_amdgcn_update_dpp(id, (int)v, 0x143, 0xc, 0xf, false));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Block-wide reductions for up to 1024 threads; `red` needs 32 floats.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  int nw = (blockDim.x + STK_WAVE - 1) / STK_WAVE;
  float r = 0.f;
  for (int i = 0; i < nw; ++i) r += red[i];
  __syncthreads();
  return r;
}
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  __syncthreads();
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  int nw = (blockDim.x + STK_WAVE - 1) / STK_WAVE;
  float r = -INFINITY;
  for (int i = 0; i < nw; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ int block_or(int v, int* red) {
  int w = __any(v != 0);
  __syncthreads();
  if (lane_id() == 0) red[wave_id()] = w;
  __syncthreads();
  int nw = (blockDim.x + STK_WAVE - 1) / STK_WAVE;
  int r = 0;
  for (int i = 0; i < nw; ++i) r |= red[i];
  __syncthreads();
  return r;
}
__device__ __forceinline__ int block_count(int v, int* red) {
  int w = __popcll(__ballot(v != 0));
  __syncthreads();
  if (lane_id() == 0) red[wave_id()] = w;
  __syncthreads();
  int nw = (blockDim.x + STK_WAVE - 1) / STK_WAVE;
  int r = 0;
  for (int i = 0; i < nw; ++i) r += red[i];
  __syncthreads();
  return r;
}

// exp(a - b) where an empty state (a == -inf) contributes exactly 0, also
// when b is -inf.
// exp(a - b), 0 for a = -inf.  The hardware exponential (2^x after one
// multiply by log2 e) is accurate to a few ulp, far inside the FP32
// softmax's own rounding.
__device__ __forceinline__ float wexp(float a, float b) {
  return a == -INFINITY ? 0.f : __expf(a - b);
}

// --------------------------------------------------------------- scans
template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v) {
  const int lane = lane_id();
#pragma unroll
  for (int off = 1; off < STK_WAVE; off <<= 1) {
    T x = __shfl_up(v, off);
    if (lane >= off) v += x;
  }
  return v;
}

// Exclusive prefix sum over the whole workgroup in thread order; `tmp`
// holds one int per wave.  Returns the exclusive prefix; *total the sum.
__device__ __forceinline__ int block_excl_scan(int v, int* tmp, int* total) {
  int inc = wave_incl_scan(v);
  const int nw = blockDim.x / STK_WAVE;
  if (lane_id() == STK_WAVE - 1) tmp[wave_id()] = inc;
  __syncthreads();
  int before = 0, all = 0;
  for (int w = 0; w < nw; ++w) {
    int x = tmp[w];
    before += w < wave_id() ? x : 0;
    all += x;
  }
  __syncthreads();
  *total = all;
  return before + inc - v;
}

// Inclusive prefix sum over the wave through DPP: row shifts by 1, 2, 4, 8
// inside each 16-lane row (lanes without a source add 0), then the row
// broadcasts of lanes 15 and 31 carry the row totals into the later rows.
// Needs every lane of the wave active.
__device__ __forceinline__ int wave_incl_scan_dpp(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);
  return v;
}

// Wave-uniform OR / AND of a 32-bit value (DPP reduction pattern of
// wave_max_u, lane 63 ends with the total).  Needs every lane active.
template <bool AND>
__device__ __forceinline__ uint32_t wave_bits_u(uint32_t v) {
  const int id = AND ? -1 : 0;
  auto step = [&](int x, int y) { return AND ? (x & y) : (x | y); };
  int x = (int)v;
  x = step(x, __builtin_amdgcn_update_dpp(id, x, 0xB1, 0xf, 0xf, false));
  x = step(x, __builtin_amdgcn_update_dpp(id, x, 0x4E, 0xf, 0xf, false));
  x = step(x, __builtin_amdgcn_update_dpp(id, x, 0x141, 0xf, 0xf, false));
  x = step(x, __builtin_amdgcn_update_dpp(id, x, 0x140, 0xf, 0xf, false));
  x = step(x, __builtin_amdgcn_update_dpp(id, x, 0x142, 0xa, 0xf, false));
  x = step(x, __builtin_amdgcn_update_dpp(id, x, 0x143, 0xc, 0xf, false));
  return (uint32_t)__builtin_amdgcn_readlane(x, 63);
}
template <bool AND>
__device__ __forceinline__ uint64_t wave_bits64_u(uint64_t v) {
  return ((uint64_t)wave_bits_u<AND>((uint32_t)(v >> 32)) << 32) | wave_bits_u<AND>((uint32_t)v);
}

// Lanes below this one.
__device__ __forceinline__ uint64_t lanemask_lt() { return (1ull << lane_id()) - 1ull; }

// Wait until every vector memory load of this wave has returned (s_waitcnt
// vmcnt(0); expcnt and lgkmcnt left free).  Placed where the outstanding
// loads are known to have returned long ago, it costs nothing and resets
// the compiler's count: loads issued afterwards under a branch then do not
// make later uses of the earlier loads wait for them (at a join the
// compiler assumes the path without those loads and waits for everything).
__device__ __forceinline__ void vm_drain() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Exclusive prefix sum over the workgroup in thread order with one barrier;
// `tmp` holds one int per wave and must not be rewritten until every thread
// has returned (use a fresh buffer or a barrier).  Needs full waves.
__device__ __forceinline__ int block_excl_scan1(int v, int* tmp, int* total) {
  const int inc = wave_incl_scan_dpp(v);
  const int nw = blockDim.x / STK_WAVE;
  if (lane_id() == STK_WAVE - 1) tmp[wave_id()] = inc;
  __syncthreads();
  int before = 0, all = 0;
  for (int w = 0; w < nw; ++w) {
    const int x = tmp[w];
    before += w < wave_id() ? x : 0;
    all += x;
  }
  *total = all;
  return before + inc - v;
}

__device__ __forceinline__ uint64_t wave_or64(uint64_t v) {
  for (int off = 1; off < STK_WAVE; off <<= 1) v |= __shfl_xor(v, off);
  return v;
}
__device__ __forceinline__ uint64_t wave_and64(uint64_t v) {
  for (int off = 1; off < STK_WAVE; off <<= 1) v &= __shfl_xor(v, off);
  return v;
}


// ------------------------------------------------ agent-scope publication
// Accesses coherent at agent scope (global_{load,store} ... sc1): a store
// goes past the XCD-local L2 to the device's coherence point, and a load
// never takes a stale line from the L2.  A producer publishes data written
// this way with wait_stores() and then a flag store; a consumer that sees the
// flag set (reading it this way) and then reads the data this way sees the
// data.  No cache-wide fence (L2 write-back) is needed, because every
// published word was itself written coherently.  (These are the code
// sequences of relaxed agent-scope atomics on gfx950.)
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float* p, float v) {
  st_agent(reinterpret_cast<uint32_t*>(p), __float_as_uint(v));
}
// two floats at an 8-byte aligned address, one store
__device__ __forceinline__ void st_agent2(float* p, float a, float b) {
  st_agent(reinterpret_cast<uint64_t*>(p),
           ((uint64_t)__float_as_uint(b) << 32) | __float_as_uint(a));
}
__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_agent(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agentf(const float* p) {
  return __uint_as_float(ld_agent(reinterpret_cast<const uint32_t*>(p)));
}
// Wait until every memory access of this wave has completed, stores
// included (gfx9 counts both in vmcnt), and keep the compiler from moving
// memory accesses across the wait.
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Longest wait for a flag, in ticks of the 100 MHz real-time counter
// (20 ms); past it the waiter records an error and goes on, so every wave
// ends whatever the flags hold.
constexpr uint64_t kSpinTicks = 2000000ull;

// Wave-level bounded wait until flag[i] != 0 for every i < cnt; false (and
// *err incremented) once `spin` ticks have passed.  Every lane returns
// together.
__device__ __forceinline__ bool wait_flags(const uint32_t* flag, int cnt, uint32_t* err,
                                           uint64_t spin = kSpinTicks) {
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  while (true) {
    int ready = 1;
    for (int i = lane_id(); i < cnt; i += STK_WAVE) ready &= ld_agent(flag + i) != 0u;
    if (__all(ready)) return true;
    if (__builtin_amdgcn_s_memrealtime() - t0 > spin) {
      if (lane_id() == 0) atomicAdd(err, 1u);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// wait_flags for flags that carry a range of key high words, each
// (max >> 16) << 16 | (min >> 16) of its chunk; also returns, in every lane,
// [hmin, hmax] covering every chunk's range (after a time-out: an empty one).
__device__ __forceinline__ bool wait_flags_range(const uint32_t* flag, int cnt, uint32_t* err,
                                                 uint64_t spin, uint32_t& hmax, uint32_t& hmin) {
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  while (true) {
    int ready = 1;
    uint32_t mx = 0u, mn = 0xffffu;
    for (int i = lane_id(); i < cnt; i += STK_WAVE) {
      const uint32_t f = ld_agent(flag + i);
      ready &= f != 0u;
      mx = (f >> 16) > mx ? (f >> 16) : mx;
      mn = (f & 0xffffu) < mn ? (f & 0xffffu) : mn;
    }
    if (__all(ready)) {
      hmax = (wave_ext_u32<true>(mx) << 16) | 0xffffu;
      hmin = wave_ext_u32<false>(mn) << 16;
      return true;
    }
    if (__builtin_amdgcn_s_memrealtime() - t0 > spin) {
      if (lane_id() == 0) atomicAdd(err, 1u);
      hmax = 0u;
      hmin = 0xffffffffu;
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

__device__ __forceinline__ bool is_bad(float x) { return !(fabsf(x) <= 3.402823466e38f); }

}  // namespace stk
