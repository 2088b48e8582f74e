// Instantiations of the one-workgroup saved / union repair (repair_fast.hpp)
// and their shape dispatch, in a translation unit of their own.
#include "repair_fast.hpp"
#include "step.hpp"

namespace stk {

template <typename T, int NCH, int UP, int RPT>
__global__ __launch_bounds__(kTailThreads) void k_repair_fast(GqaRepairArgs a) {
  // a KV group's heads on one XCD: tiles that several of them miss come
  // from HBM once
  repair_fast_head<T, NCH, UP, RPT>(a, xcd_remap(blockIdx.x, gridDim.x));
}

namespace {

template <typename T, int NCH, int UP>
void launch_t(const GqaRepairArgs& g, int rpt, hipStream_t st) {
  const dim3 grid(g.kv.hq), block(kTailThreads);
  if (rpt == 4) hipLaunchKernelGGL((k_repair_fast<T, NCH, UP, 4>), grid, block, 0, st, g);
  else hipLaunchKernelGGL((k_repair_fast<T, NCH, UP, 16>), grid, block, 0, st, g);
}

}  // namespace

int launch_repair_fast(const GqaRepairArgs& g, int dtype, hipStream_t st) {
  const uintptr_t align = reinterpret_cast<uintptr_t>(g.kv.q) |
                          reinterpret_cast<uintptr_t>(g.kv.k) |
                          reinterpret_cast<uintptr_t>(g.kv.v) | reinterpret_cast<uintptr_t>(g.pu);
  if (dtype != DT_BF16 && dtype != DT_F16) return 1;
  const int nch = tok_nch(dtype, g.kv.d, g.kv.b, align);
  const int up = tok_up(g.kv.b);
  const int rpt = repair_fast_rpt(g.sp, g.kv.d);
  if (!nch || g.kv.b != 16 * up || g.kv.n > kTailMapN || g.sa > kTailMaxK ||
      g.sp > kTailMaxK || !rpt || (nch == 8 && up == 2 && rpt == 16))   // the last spills
    return 1;
  STK_DISPATCH_STEP(dtype, nch, {
    if (up == 1) launch_t<T, NCH, 1>(g, rpt, st);
    else launch_t<T, NCH, 2>(g, rpt, st);
  });
  return stk_check_launch("k_repair_fast");
}

}  // namespace stk
