// Instantiations of the direct-activation W8A8 kernel (16-row token tiles), every BLOCK_N and
// both weight layouts.
#include "w8a8_tiles.hpp"

namespace specq {

const void* w8a8_rk_fn(int bnsel, int layout) {
  switch (bnsel * 2 + layout) {
    case 0: return w8a8_rk_pick<0, 0>();
    case 1: return w8a8_rk_pick<0, 1>();
    case 2: return w8a8_rk_pick<1, 0>();
    case 3: return w8a8_rk_pick<1, 1>();
    case 4: return w8a8_rk_pick<2, 0>();
    case 5: return w8a8_rk_pick<2, 1>();
    case 6: return w8a8_rk_pick<3, 0>();
    case 7: return w8a8_rk_pick<3, 1>();
    default: return nullptr;
  }
}

}  // namespace specq
