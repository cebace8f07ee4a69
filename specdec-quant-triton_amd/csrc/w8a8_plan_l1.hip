// Instantiation of the plan-mode W8A8 launch with several tilings, weight layout 1.
#include "w8a8_plan.hpp"

namespace specq {

const void* w8a8_plan_fn_l1(int variant) {
  return variant ? reinterpret_cast<const void*>(&w8a8_plan_kernel<1, 1>)
                 : reinterpret_cast<const void*>(&w8a8_plan_kernel<1, 0>);
}

}  // namespace specq
