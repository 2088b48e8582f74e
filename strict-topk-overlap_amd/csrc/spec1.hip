// The hybrid speculation in one launch: kernels.speculate(mode='hybrid')
// (strict_topk/kernels.py:450-477, _group :94-117) as one grid of 256-thread
// workgroups in two roles, in launch order:
//   states    one wave per (query head, predicted slot): the block's
//             softmax state (states_tok.hpp), stored agent-coherent; once the
//             wave's stores have completed, the item's flag;
//   grouping  one workgroup per query head: waits for its head's item flags,
//             clears them, then groups the head's states in one round trip
//             (group.hpp) with agent-coherent loads.
// The grouping starts as soon as its head's states are published instead of
// behind a kernel boundary; the arithmetic is that of k_states_tok followed
// by k_hybrid_group1, so the results are the same bits.  The flags live in
// the stream's slot (flags.hpp); a wait past its limit makes the head's
// grouping outputs NaN.
#include "flags.hpp"
#include "group.hpp"
#include "states_tok.hpp"
#include "api.hpp"

namespace stk {

struct Spec1Args {
  StatesArgs st;       // st.tflag: [hq * s] item flags
  GroupArgs g;
  uint32_t* err;       // the slot's time-out counter
  uint64_t spin;       // longest wait
  int T;               // states workgroups (four items each)
};

template <typename T, int NCH, int UP, typename I>
__global__ __launch_bounds__(256, 4) void k_spec1(Spec1Args a) {
  const int b = blockIdx.x;
  if (b < a.T) {
    states_tok_wg<T, NCH, UP, I, true, false, true>(a.st, xcd_remap(b, a.T));
    return;
  }
  // a head's states are items h * s .. h * s + s - 1: the same XCD as this
  // workgroup when the grid's roles split evenly over the XCDs
  const int h = xcd_remap(b - a.T, a.g.h);
  __shared__ int s_fail;
  if (threadIdx.x == 0) s_fail = 0;
  __syncthreads();
  uint32_t* flag = a.st.tflag + (size_t)h * a.g.s;
  const bool ok = wait_flags(flag, a.g.s, a.err, a.spin);
  if (!ok && lane_id() == 0) atomicOr(&s_fail, 1);
  __syncthreads();
  // every wave is past its wait: the flags are clear again for the next launch
  for (int i = threadIdx.x; i < a.g.s; i += blockDim.x) st_agent(flag + i, 0u);
  group1_head<true>(a.g, h, s_fail != 0);
}

}  // namespace stk

using namespace stk;

int launch_spec1(const void* q, const void* k, const void* v, int dtype, int hq, int hkv, int n,
                 int b, int d, const void* pred, int pred_dtype, int s, float tau, float* m,
                 float* l, float* u, uint8_t* high, float* lm, float* ll, float* lu, float* labs,
                 hipStream_t st) {
  if (!flag_one_launch()) return 1;
  if (dtype != DT_BF16 && dtype != DT_F16) return 1;
  if ((b != 16 && b != 32) || (d != 64 && d != 128) || s < 1) return 1;
  if (pred_dtype != IT_I32 && pred_dtype != IT_I64) return 1;
  const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(u);
  if (!tok_nch(dtype, d, b, align) || !group1_covers(s, d, u, lu, labs)) return 1;
  uint32_t* flags = nullptr;
  const int rc = flag_slot(st, (size_t)hq * s, true, &flags);
  if (rc) return rc;
  if (!flags) return 1;
  Spec1Args a{};
  a.st.q = q; a.st.k = k; a.st.v = v; a.st.ids = pred; a.st.itype = pred_dtype;
  a.st.hq = hq; a.st.hkv = hkv; a.st.n = n; a.st.b = b; a.st.d = d; a.st.s = s;
  a.st.m = m; a.st.l = l; a.st.u = u;
  a.st.tflag = flags;
  a.st.drop = flag_drop();
  a.g = GroupArgs{m, l, u, hq, s, d, tau, high, lm, ll, lu, labs};
  a.err = flags + kFlagSlotWords - 1;
  a.spin = flag_spin();
  a.T = (int)(((int64_t)hq * s + 3) / 4);
  const dim3 grid(a.T + hq), block(256);
  const bool i64 = pred_dtype == IT_I64;
#define STK_SPEC1(TT, NCHV, UPV)                                                               \
  do {                                                                                         \
    if (i64) hipLaunchKernelGGL((k_spec1<TT, NCHV, UPV, int64_t>), grid, block, 0, st, a);     \
    else hipLaunchKernelGGL((k_spec1<TT, NCHV, UPV, int32_t>), grid, block, 0, st, a);         \
  } while (0)
#define STK_SPEC1_T(TT)                                                                        \
  do {                                                                                         \
    if (d == 64 && b == 16) STK_SPEC1(TT, 2, 1);                                               \
    else if (d == 64) STK_SPEC1(TT, 2, 2);                                                     \
    else if (b == 16) STK_SPEC1(TT, 4, 1);                                                     \
    else STK_SPEC1(TT, 4, 2);                                                                  \
  } while (0)
  if (dtype == DT_BF16) STK_SPEC1_T(bf16s);
  else STK_SPEC1_T(f16s);
#undef STK_SPEC1_T
#undef STK_SPEC1
  return stk_check_launch("k_spec1");
}
