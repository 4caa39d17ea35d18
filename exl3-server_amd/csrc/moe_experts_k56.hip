// Expert kernel instantiations for codebook widths K = 5 and 6 (moe_experts.hpp), in a
// translation unit of their own so that the widths compile in parallel.
#include "moe_experts.hpp"

namespace exl3h {

exl3_status launch_expert_k56(int K, int cb, int pd, int which, dim3 ub, hipStream_t st, const MoeArgs &a,
                              int shared_mode, int dense_arg) {
  if (K == 5) return launch_expert_k<5>(cb, pd, which, ub, st, a, shared_mode, dense_arg);
  if (K == 6) return launch_expert_k<6>(cb, pd, which, ub, st, a, shared_mode, dense_arg);
  return fail(EXL3_ERR_INVALID, "K out of range");
}

}  // namespace exl3h
