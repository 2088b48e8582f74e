// Instantiations of the paged saved / serial tail (k_tail over a page pool), in a translation unit of
// their own so that the large kernels compile in parallel (step_launch.hpp).
#include "step_launch.hpp"

int stk::launch_tail_pg(int dtype, const TailArgs& t, const StepShape& s, hipStream_t st) {
  return launch::tail<true>(dtype, t, s, st);
}
