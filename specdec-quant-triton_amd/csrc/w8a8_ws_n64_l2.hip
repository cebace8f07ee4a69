// Instantiations of the LDS-staged-activation W8A8 kernel: BLOCK_N = 64, weight layout 2
// (packed INT4 fragments of W4A8), token tiles of 2 .. 19 x 16 rows.
#include "w8a8_tiles.hpp"

namespace specq {

const void* w8a8_ws_fn_n64_l2(int mt) {
  switch (mt) {
    case 2: return w8a8_ws_pick<2, 2, 2>();
    case 3: return w8a8_ws_pick<3, 2, 2>();
    case 4: return w8a8_ws_pick<4, 2, 2>();
    case 5: return w8a8_ws_pick<5, 2, 2>();
    case 6: return w8a8_ws_pick<6, 2, 2>();
    case 7: return w8a8_ws_pick<7, 2, 2>();
    case 8: return w8a8_ws_pick<8, 2, 2>();
    case 9: return w8a8_ws_pick<9, 2, 2>();
    case 10: return w8a8_ws_pick<10, 2, 2>();
    case 11: return w8a8_ws_pick<11, 2, 2>();
    case 12: return w8a8_ws_pick<12, 2, 2>();
    case 13: return w8a8_ws_pick<13, 2, 2>();
    case 14: return w8a8_ws_pick<14, 2, 2>();
    case 15: return w8a8_ws_pick<15, 2, 2>();
    case 16: return w8a8_ws_pick<16, 2, 2>();
    case 17: return w8a8_ws_pick<17, 2, 2>();
    case 18: return w8a8_ws_pick<18, 2, 2>();
    case 19: return w8a8_ws_pick<19, 2, 2>();
    default: return nullptr;
  }
}

}  // namespace specq
