// Instantiations of the one-launch speculative step (k_step1, step1.hpp) and
// their shape dispatch, in a translation unit of their own so that the large
// kernels compile in parallel.
#include "step1.hpp"

namespace stk {

bool step1_covers(int dtype, int hq, int hkv, int b, int d, const StepShape& s) {
  return (dtype == DT_BF16 || dtype == DT_F16) && b == 32 && (d == 64 || d == 128) &&
         hq / hkv <= 4 && s.one && s.up == 2 && s.rpt == 4;
}

namespace {

template <typename T, int NCH>
int launch_t(const Step1Args& a, const StepShape& s, hipStream_t st) {
  const dim3 grid(a.S + a.T + a.H), block(kStep1Threads);
  if (s.kpt == 4) hipLaunchKernelGGL((k_step1<T, NCH, 4, 4>), grid, block, 0, st, a);
  else if (s.kpt == 8) hipLaunchKernelGGL((k_step1<T, NCH, 8, 4>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((k_step1<T, NCH, 16, 4>), grid, block, 0, st, a);
  return stk_check_launch("k_step1");
}

}  // namespace

int launch_step1(int dtype, const FrontArgs& f, const TailArgs& t, const StepShape& s,
                 uint32_t* ctl, size_t cap, uint32_t* err, uint64_t spin, int drop,
                 hipStream_t st) {
  if (!step1_covers(dtype, t.kv.hq, t.kv.hkv, t.kv.b, t.kv.d, s)) return 1;
  Step1Args a{};
  a.f = f;
  a.t = t;
  const int hq = t.kv.hq, n = t.kv.n;
  a.f.sc.chunks = (n + kStep1Blocks - 1) / kStep1Blocks;
  a.S = t.kv.hkv * a.f.sc.chunks;
  a.T = (int)(((int64_t)hq * t.sp + kStep1Waves - 1) / kStep1Waves);
  a.H = hq;
  // each head's chunk flags on a 128-byte line of their own when the slot
  // holds that layout, else packed
  const int line = (a.f.sc.chunks + 31) & ~31;
  a.f.sc.fstride = (size_t)hq * (line + t.sp) <= cap ? line : a.f.sc.chunks;
  a.f.sc.sflag = ctl;
  a.f.st.tflag = ctl + (size_t)hq * a.f.sc.fstride;
  a.err = err;
  a.spin = spin;
  a.f.sc.drop = a.f.st.drop = drop;
  if (dtype == DT_BF16) {
    return t.kv.d == 64 ? launch_t<bf16s, 2>(a, s, st) : launch_t<bf16s, 4>(a, s, st);
  }
  return t.kv.d == 64 ? launch_t<f16s, 2>(a, s, st) : launch_t<f16s, 4>(a, s, st);
}

}  // namespace stk
