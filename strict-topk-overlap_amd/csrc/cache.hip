// Host-backed KV cache: the decode step over a pinned host page pool with a
// device-resident working set per (request, KV head).
//
// Reference: docs/hisparse_integration.md:11-27 (HiSparse keeps the full KV
// in a pinned host pool and a hot device buffer per request; after the
// selector has produced the logical top-K, swap-in finds the resident hits,
// updates the LRU, copies the missing blocks in and returns the device slot
// table for attention; the first phase speculates only on resident
// predicted blocks, P n R, and repairs the selected set A from the device
// slots after swap-in).  That design targets SGLang's HiSparse; here it is
// the native layout of this library:
//
//   host pool (pinned, read by the GPU in place): host_k, host_v [HP, B, D]
//   host_table [R, Hkv, NB] int32      host page of logical block j
//   lo/hi pages [HP, D] on the device  every block's bounds (the scorer
//                                      scores every block, resident or not)
//   device slots k_slots, v_slots [R * Hkv * C, B, D]: group g = r * Hkv +
//                                      kvh owns slots [g * C, g * C + C)
//   table [R, Hkv, NB] int32           device slot of block j, or -1
//   slot_block [R * Hkv * C]           block held by a slot, or -1
//   slot_stamp [R * Hkv * C]           step of the slot's last use (LRU)
//   clock [1]                          step counter, advanced once a step
//
// One step is five launches on one stream:
//   k_front (paged)  bound scores of every block (bounds table = host_table)
//                    || prediction states of the resident predicted blocks
//                    (P n R: a predicted block without a slot gets the empty
//                    state, and no LRU update, no copy);
//   k_cache_select   top-K of every (request, head) -> the selected IDs, and
//                    the clock advances;
//   k_swap_in        per group: the union of its heads' selected blocks;
//                    resident ones are stamped, missing ones take the least
//                    recently used slots not needed this step (free slots
//                    first), the table is updated and the copies listed;
//                    H2D bytes are counted;
//   k_swap_copy      the listed host pages into their slots, 16 workgroups
//                    per group with several 16-byte loads in flight per
//                    thread (host reads cross PCIe: their latency needs many
//                    bytes in flight);
//   k_tail (paged)   the repair: a predicted block with a state that is
//                    selected is a hit, every other selected block (A \ P
//                    and A n (P \ R)) is computed from its slot.
// Capacity: C >= G * K slots per group, so that every selected block fits.
#include "step_launch.hpp"

using namespace stk;

namespace {

constexpr int kSwapThreads = 256;
constexpr int kMaxSlots = 1024;     // slots per group
constexpr int kMaxNeed = 1024;      // distinct selected blocks per group
constexpr int kSlotsPerThread = kMaxSlots / kSwapThreads;

struct SelArgs {
  const uint64_t* keys;   // [R * Hq, NB]
  int hq, hkv, nb, k;     // hq / hkv flattened over the batch
  Paging pg;
  int32_t* ids;           // [R * Hq, K], -1 past a short request's blocks
  int32_t* clock;
};

template <int KPT>
__global__ __launch_bounds__(kTailThreads) void k_cache_select(SelArgs a) {
  __shared__ TopkBinsLds tb;
  __shared__ int s_scan[kTailWaves];
  const int h = blockIdx.x, tid = threadIdx.x;
  const int kv = h / (a.hq / a.hkv);
  uint64_t key[KPT];
  topk_load<KPT>(a.keys + (size_t)h * a.nb, a.nb, key);
  const int n = pg_blocks(a.pg, kv, a.nb);
  const int kk = a.k < n ? a.k : n;
  uint32_t flags = 0;
  if (kk > 0) flags = topk_bins_flags<KPT>(key, n, kk, tb, [] {});
  int total;
  int pos = block_excl_scan1(__popc(flags), s_scan, &total);
#pragma unroll
  for (int i = 0; i < KPT; ++i)
    if ((flags >> i) & 1u) a.ids[(size_t)h * a.k + pos++] = tid * KPT + i;
  for (int i = kk + tid; i < a.k; i += kTailThreads) a.ids[(size_t)h * a.k + i] = -1;
  if (h == 0 && tid == 0) atomicAdd(a.clock, 1);
}

constexpr int kCopyWGs = 16;        // copy workgroups per group
constexpr int kCopyUnroll = 4;      // 16-byte loads in flight per thread

struct SwapArgs {
  const int32_t* ids;     // [R * Hq, K]
  int g, k, nb, hkv_req, c;   // heads per group, K, NB, KV heads per request, slots per group
  int b, d, esize;
  const int32_t* nblk;    // [R]
  const void* host_k; const void* host_v;
  const int32_t* host_table;   // [R * Hkv, NB]
  int host_pages;
  void* k_slots; void* v_slots;
  int32_t* table;         // [R * Hkv, NB]
  int32_t* slot_block;    // [R * Hkv * C]
  int32_t* slot_stamp;
  const int32_t* clock;
  unsigned long long* h2d;
  int32_t* nlist;         // [R * Hkv] pages to copy per group
  int32_t* src;           // [R * Hkv, kMaxNeed] host pages
  int32_t* dst;           // [R * Hkv, kMaxNeed] device slots
};

// One workgroup per group (request, KV head).
__global__ __launch_bounds__(kSwapThreads) void k_swap_in(SwapArgs a) {
  __shared__ uint32_t need[kTailMapN / 32];
  __shared__ int loads[kMaxNeed];
  __shared__ int loads_hp[kMaxNeed];   // the listed blocks' host pages
  __shared__ int vict[kMaxNeed];
  __shared__ TopkLds tl;
  __shared__ int nload;
  const int grp = blockIdx.x, tid = threadIdx.x;
  const int r = grp / a.hkv_req;
  const int n = a.nblk[r] < a.nb ? (a.nblk[r] < 0 ? 0 : a.nblk[r]) : a.nb;
  const int words = (a.nb + 31) / 32;
  for (int w = tid; w < words; w += kSwapThreads) need[w] = 0u;
  for (int x = tid; x < kMaxNeed; x += kSwapThreads) vict[x] = -1;
  if (tid == 0) nload = 0;
  const int now = *a.clock;
  int32_t* trow = a.table + (size_t)grp * a.nb;
  const int32_t* hrow = a.host_table + (size_t)grp * a.nb;
  const size_t s0 = (size_t)grp * a.c;
  // this thread's slots' blocks and stamps, for the victim keys below (the
  // stamps written in between belong to needed slots, whose keys ignore them)
  int sblk[kSlotsPerThread], sstamp[kSlotsPerThread];
#pragma unroll
  for (int i = 0; i < kSlotsPerThread; ++i) {
    const int sl = tid * kSlotsPerThread + i;
    sblk[i] = sl < a.c ? a.slot_block[s0 + sl] : -1;
    sstamp[i] = sl < a.c ? a.slot_stamp[s0 + sl] : 0;
  }
  __syncthreads();
  // the union of the group's selected blocks: the thread that sets a block's
  // bit handles it, its slot and host page requested together (one round
  // trip for the whole union).  Resident blocks are stamped, missing ones
  // listed; a block with no valid host page is neither (it stays
  // non-resident: the tail gives it the empty state, as the paged steps do
  // for an invalid page).
  const int32_t* gids = a.ids + (size_t)grp * a.g * a.k;
  for (int x = tid; x < a.g * a.k; x += kSwapThreads) {
    const int id = gids[x];
    const bool in = id >= 0 && id < n;
    const uint32_t bit = 1u << (in ? (id & 31) : 0);
    const bool first = in && !(atomicOr(&need[in ? id >> 5 : 0], in ? bit : 0u) & bit);
    const int j = first ? id : 0;
    const int s = trow[j];
    const int hp = hrow[j];
    if (first) {
      if (s >= 0) {
        a.slot_stamp[s] = now;
      } else if (hp >= 0 && hp < a.host_pages) {
        const int y = atomicAdd(&nload, 1);
        if (y < kMaxNeed) {
          loads[y] = j;
          loads_hp[y] = hp;
        }
      }
    }
  }
  __syncthreads();
  const int nl = nload < kMaxNeed ? nload : kMaxNeed;
  if (tid == 0) a.nlist[grp] = nl;
  if (nl == 0) return;   // the whole selection is resident
  // victims: the nl slots whose block is not needed this step, free slots
  // first, then least recently used (ties to the lower slot): the largest
  // keys ~(stamp + 1, slot) by the radix select, a needed slot keyed 0
  uint64_t vkey[kSlotsPerThread];
#pragma unroll
  for (int i = 0; i < kSlotsPerThread; ++i) {
    const int s = tid * kSlotsPerThread + i;
    const int blk = sblk[i];
    const bool busy = blk >= 0 && blk < a.nb && ((need[blk >> 5] >> (blk & 31)) & 1u);
    const uint64_t stamp = blk < 0 ? 0ull : (uint64_t)(uint32_t)(sstamp[i] + 1);
    vkey[i] = busy ? 0ull : ~((stamp << 20) | (uint64_t)s);
  }
  topk_select_keys<kSlotsPerThread>(vkey, a.c, nl, tl, [&](int pos, int s, int i) {
    if (vkey[i] == 0ull) return;   // a needed slot (C >= G * K rules this out)
    const int j = loads[pos];
    const int old = sblk[i];
    if (old >= 0 && old < a.nb) trow[old] = -1;
    a.slot_block[s0 + s] = j;
    a.slot_stamp[s0 + s] = now;
    trow[j] = (int)(s0 + s);
    vict[pos] = (int)(s0 + s);
  });
  __syncthreads();
  // the copy list: host page and device slot of each listed block (a block
  // left without a slot, which C >= G * K rules out, is copied nowhere and
  // not counted)
  __shared__ int ncopy;
  if (tid == 0) ncopy = 0;
  __syncthreads();
  for (int x = tid; x < nl; x += kSwapThreads) {
    const int hp = loads_hp[x];
    const bool ok = hp >= 0 && hp < a.host_pages && vict[x] >= 0;
    a.src[(size_t)grp * kMaxNeed + x] = ok ? hp : -1;
    a.dst[(size_t)grp * kMaxNeed + x] = ok ? vict[x] : -1;
    const int c = __popcll(__ballot(ok));
    if (lane_id() == __ffsll((long long)__ballot(1)) - 1) atomicAdd(&ncopy, c);
  }
  __syncthreads();
  const int chunks = a.b * a.d * a.esize / 16;   // 16-byte chunks per page
  if (tid == 0) atomicAdd(a.h2d, (unsigned long long)ncopy * 2ull * chunks * 16ull);
}

// The listed pages: workgroup (group, part) copies pages part, part + 16,
// ... of its group's list, K then V, every thread keeping kCopyUnroll
// 16-byte host loads in flight before its stores.
__global__ __launch_bounds__(kSwapThreads) void k_swap_copy(SwapArgs a) {
  const int grp = blockIdx.x / kCopyWGs, part = blockIdx.x % kCopyWGs;
  const int nl = a.nlist[grp];
  const int chunks = a.b * a.d * a.esize / 16;
  const uint4* hk = reinterpret_cast<const uint4*>(a.host_k);
  const uint4* hv = reinterpret_cast<const uint4*>(a.host_v);
  uint4* dk = reinterpret_cast<uint4*>(a.k_slots);
  uint4* dv = reinterpret_cast<uint4*>(a.v_slots);
  for (int x = part; x < nl; x += kCopyWGs) {
    const int hp = a.src[(size_t)grp * kMaxNeed + x], sl = a.dst[(size_t)grp * kMaxNeed + x];
    if (hp < 0 || sl < 0) continue;
    const size_t so = (size_t)hp * chunks, dof = (size_t)sl * chunks;
    for (int c0 = threadIdx.x; c0 < 2 * chunks; c0 += kSwapThreads * kCopyUnroll) {
      uint4 buf[kCopyUnroll];
#pragma unroll
      for (int u = 0; u < kCopyUnroll; ++u) {
        const int c = c0 + u * kSwapThreads;
        const int cc = c < 2 * chunks ? c : 0;
        buf[u] = cc < chunks ? hk[so + cc] : hv[so + cc - chunks];
      }
#pragma unroll
      for (int u = 0; u < kCopyUnroll; ++u) {
        const int c = c0 + u * kSwapThreads;
        if (c < chunks) dk[dof + c] = buf[u];
        else if (c < 2 * chunks) dv[dof + c - chunks] = buf[u];
      }
    }
  }
}

}  // namespace

extern "C" {

// The paged step's workspace, then the copy lists (count, host pages and
// slots of every group).
static size_t cache_lists_bytes(int requests, int hkv) {
  return stk_align((size_t)requests * hkv * (1 + 2 * kMaxNeed) * sizeof(int32_t));
}

STK_API size_t stk_cache_workspace_bytes(int requests, int hq, int hkv, int nb) {
  if (requests <= 0 || hq <= 0 || hkv <= 0 || nb <= 0) return 0;
  return stk_align(stk_paged_workspace_bytes(requests, hq, nb)) + cache_lists_bytes(requests, hkv);
}

STK_API int stk_cache_step(const void* q, int dtype, int requests, int hq, int hkv, int nb, int b,
                           int d, void* k_slots, void* v_slots, int slots_per_group,
                           const void* host_k, const void* host_v, int host_pages,
                           const void* lo_pages, const void* hi_pages, int bounds_dtype,
                           const int32_t* host_table, int32_t* table, int32_t* slot_block,
                           int32_t* slot_stamp, int32_t* clock, const int32_t* nblocks,
                           const int32_t* ntokens, int topk, const int32_t* predicted, int sp,
                           int32_t* selected, float* m, float* l, float* u, float* out,
                           unsigned long long* h2d_bytes, void* workspace,
                           size_t workspace_bytes, void* stream) {
  STK_REQUIRE(q && k_slots && v_slots && host_k && host_v && lo_pages && hi_pages &&
                  host_table && table && slot_block && slot_stamp && clock && nblocks &&
                  selected && out && h2d_bytes && workspace,
              "null pointer");
  STK_REQUIRE(requests >= 1 && hq >= 1 && hkv >= 1 && hq % hkv == 0 && nb >= 1 && b >= 1 &&
                  d >= 1 && host_pages >= 1,
              "bad shape");
  STK_REQUIRE(dtype == DT_BF16 || dtype == DT_F16, "the cache step takes bf16 or fp16 K/V");
  STK_REQUIRE(stk_bounds_ok(dtype, bounds_dtype),
              "lo and hi pages must be FP32 or the pages' 16-bit type");
  STK_REQUIRE(topk >= 1 && topk <= kTailMaxK, "topk must be in [1, 256]");
  STK_REQUIRE(sp >= 0 && sp <= kTailMaxK, "the predicted width must be in [0, 256]");
  STK_REQUIRE(sp == 0 || (predicted && m && l && u), "null pointer");
  STK_REQUIRE(nb <= kTailMapN, "at most 8192 blocks per request");
  const int G = hq / hkv;
  STK_REQUIRE(slots_per_group >= G * topk && slots_per_group <= kMaxSlots,
              "slots per (request, KV head) must be in [G * topk, 1024]");
  STK_REQUIRE((b * d * 2) % 16 == 0, "a page must be a whole number of 16-byte chunks");
  STK_REQUIRE((int64_t)requests * hkv * slots_per_group <= 0x7fffffff, "too many slots");
  STK_REQUIRE(workspace_bytes >= stk_cache_workspace_bytes(requests, hq, hkv, nb),
              "workspace too small");
  const int R = requests;
  const int hqa = R * hq, hkva = R * hkv;
  const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_slots) |
                          reinterpret_cast<uintptr_t>(v_slots) |
                          reinterpret_cast<uintptr_t>(host_k) |
                          reinterpret_cast<uintptr_t>(host_v) |
                          reinterpret_cast<uintptr_t>(lo_pages) |
                          reinterpret_cast<uintptr_t>(hi_pages) | reinterpret_cast<uintptr_t>(u);
  StepShape s{};
  const char* why = plan_step(dtype, hqa, hkva, nb, b, d, topk < nb ? topk : nb,
                              sp > 0 ? sp : 1, IT_I32, align, &s);
  STK_REQUIRE(why == nullptr, why ? why : "");
  uint64_t* keys = static_cast<uint64_t*>(workspace);
  const int pages = R * hkv * slots_per_group;
  FrontArgs f = make_front_args(q, k_slots, v_slots, dtype, hqa, hkva, nb, b, d, lo_pages,
                                hi_pages, bounds_dtype != 0, predicted, sp, m, l, u, keys, s);
  f.pg = Paging{table, nblocks, hkv, pages, ntokens, host_table, host_pages};
  hipStream_t st = (hipStream_t)stream;
  int rc = launch_front_pg(dtype, f, s, st);
  if (rc) return rc;
  SelArgs sa{keys, hqa, hkva, nb, topk, f.pg, selected, clock};
  const dim3 tgrid(hqa), tblock(kTailThreads);
  if (s.kpt == 4) hipLaunchKernelGGL(k_cache_select<4>, tgrid, tblock, 0, st, sa);
  else if (s.kpt == 8) hipLaunchKernelGGL(k_cache_select<8>, tgrid, tblock, 0, st, sa);
  else hipLaunchKernelGGL(k_cache_select<16>, tgrid, tblock, 0, st, sa);
  rc = stk_check_launch("k_cache_select");
  if (rc) return rc;
  int32_t* lists = reinterpret_cast<int32_t*>(
      static_cast<char*>(workspace) + stk_align(stk_paged_workspace_bytes(requests, hq, nb)));
  SwapArgs w{selected, G, topk, nb, hkv, slots_per_group, b, d, 2, nblocks, host_k, host_v,
             host_table, host_pages, k_slots, v_slots, table, slot_block, slot_stamp, clock,
             h2d_bytes, lists, lists + hkva, lists + hkva + (size_t)hkva * kMaxNeed};
  hipLaunchKernelGGL(k_swap_in, dim3(hkva), dim3(kSwapThreads), 0, st, w);
  rc = stk_check_launch("k_swap_in");
  if (rc) return rc;
  hipLaunchKernelGGL(k_swap_copy, dim3(hkva * kCopyWGs), dim3(kSwapThreads), 0, st, w);
  rc = stk_check_launch("k_swap_copy");
  if (rc) return rc;
  // with no predicted rows (the serial path) the tail's always-issued loads
  // of slot 0 read a stand-in past the keys (their values are discarded)
  const void* dummy = static_cast<char*>(workspace) +
                      stk_align((size_t)requests * hq * nb * sizeof(uint64_t));
  TailArgs t{};
  t.kv = KV{q, k_slots, v_slots, hqa, hkva, nb, b, d};
  t.keys = keys; t.k = topk; t.ids = selected;
  t.p = sp ? predicted : static_cast<const int32_t*>(dummy); t.sp = sp;
  t.pm = sp ? m : static_cast<const float*>(dummy);
  t.pl = sp ? l : static_cast<const float*>(dummy);
  t.pu = sp ? u : static_cast<const float*>(dummy);
  t.uni = 0; t.out = out;
  t.pg = f.pg;
  return launch_tail_pg(dtype, t, s, st);
}

}  // extern "C"
