// Instantiation of the plan-mode W4A16 launch with several tilings, weight layout 2.
#include "w4a16_plan.hpp"

namespace specq {

const void* w4a16_plan_fn_l2() { return reinterpret_cast<const void*>(&w4a16_plan_kernel<2>); }

}  // namespace specq
