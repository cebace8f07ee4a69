// Instantiation of the plan-mode W8A8 launch with several tilings, weight layout 0.
#include "w8a8_plan.hpp"

namespace specq {

const void* w8a8_plan_fn_l0(int variant) {
  return variant ? reinterpret_cast<const void*>(&w8a8_plan_kernel<0, 1>)
                 : reinterpret_cast<const void*>(&w8a8_plan_kernel<0, 0>);
}

}  // namespace specq
