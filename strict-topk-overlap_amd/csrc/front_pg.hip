// Instantiations of the paged front (k_front over a page pool), in a translation unit of
// their own so that the large kernels compile in parallel (step_launch.hpp).
#include "step_launch.hpp"

int stk::launch_front_pg(int dtype, const FrontArgs& f, const StepShape& s, hipStream_t st) {
  return launch::front<true>(dtype, f, s, st);
}
