// Instantiations of the paged signed tail (k_stail over a page pool), in a translation unit of
// their own so that the large kernels compile in parallel (step_launch.hpp).
#include "step_launch.hpp"

int stk::launch_stail_pg(int dtype, const STailArgs& t, const StepShape& s, hipStream_t st) {
  return launch::stail<true>(dtype, t, s, st);
}
