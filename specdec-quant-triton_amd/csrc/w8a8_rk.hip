// Instantiations of the direct-activation W8A8 kernel (16-row token tiles), every BLOCK_N and
// every weight layout (0 row-major, 1 packed int8, 2 packed INT4 of W4A8).
#include "w8a8_tiles.hpp"

namespace specq {

const void* w8a8_rk_fn(int bnsel, int layout) {
  switch (bnsel * 3 + layout) {
    case 0: return w8a8_rk_pick<0, 0>();
    case 1: return w8a8_rk_pick<0, 1>();
    case 2: return w8a8_rk_pick<0, 2>();
    case 3: return w8a8_rk_pick<1, 0>();
    case 4: return w8a8_rk_pick<1, 1>();
    case 5: return w8a8_rk_pick<1, 2>();
    case 6: return w8a8_rk_pick<2, 0>();
    case 7: return w8a8_rk_pick<2, 1>();
    case 8: return w8a8_rk_pick<2, 2>();
    case 9: return w8a8_rk_pick<3, 0>();
    case 10: return w8a8_rk_pick<3, 1>();
    case 11: return w8a8_rk_pick<3, 2>();
    default: return nullptr;
  }
}

}  // namespace specq
