// Instantiations of the dense fused step's tail (k_tail), in a translation unit of
// their own so that the large kernels compile in parallel (step_launch.hpp).
#include "step_launch.hpp"

int stk::launch_tail(int dtype, const TailArgs& t, const StepShape& s, hipStream_t st) {
  return launch::tail<false>(dtype, t, s, st);
}
