// Instantiations of the plan-mode paged attention launch (runtime row blocks), head dim 64.
#include "paged_attn.hpp"

namespace specq {

const void* attn_plan_fn_d64(int rb_max, int fp32) {
  switch (rb_max * 2 + fp32) {
    case 4: return reinterpret_cast<const void*>(&paged_attn_plan_kernel<64, 2, _Float16>);
    case 5: return reinterpret_cast<const void*>(&paged_attn_plan_kernel<64, 2, float>);
    case 6: return reinterpret_cast<const void*>(&paged_attn_plan_kernel<64, 3, _Float16>);
    case 7: return reinterpret_cast<const void*>(&paged_attn_plan_kernel<64, 3, float>);
    case 8: return reinterpret_cast<const void*>(&paged_attn_plan_kernel<64, 4, _Float16>);
    case 9: return reinterpret_cast<const void*>(&paged_attn_plan_kernel<64, 4, float>);
  }
  return nullptr;
}

}  // namespace specq
