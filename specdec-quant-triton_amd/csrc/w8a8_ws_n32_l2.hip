// Instantiations of the LDS-staged-activation W8A8 kernel: BLOCK_N = 32, weight layout 2
// (packed INT4 fragments of W4A8), token tiles of 2 .. 19 x 16 rows.
#include "w8a8_tiles.hpp"

namespace specq {

const void* w8a8_ws_fn_n32_l2(int mt) {
  switch (mt) {
    case 2: return w8a8_ws_pick<2, 1, 2>();
    case 3: return w8a8_ws_pick<3, 1, 2>();
    case 4: return w8a8_ws_pick<4, 1, 2>();
    case 5: return w8a8_ws_pick<5, 1, 2>();
    case 6: return w8a8_ws_pick<6, 1, 2>();
    case 7: return w8a8_ws_pick<7, 1, 2>();
    case 8: return w8a8_ws_pick<8, 1, 2>();
    case 9: return w8a8_ws_pick<9, 1, 2>();
    case 10: return w8a8_ws_pick<10, 1, 2>();
    case 11: return w8a8_ws_pick<11, 1, 2>();
    case 12: return w8a8_ws_pick<12, 1, 2>();
    case 13: return w8a8_ws_pick<13, 1, 2>();
    case 14: return w8a8_ws_pick<14, 1, 2>();
    case 15: return w8a8_ws_pick<15, 1, 2>();
    case 16: return w8a8_ws_pick<16, 1, 2>();
    case 17: return w8a8_ws_pick<17, 1, 2>();
    case 18: return w8a8_ws_pick<18, 1, 2>();
    case 19: return w8a8_ws_pick<19, 1, 2>();
    default: return nullptr;
  }
}

}  // namespace specq
