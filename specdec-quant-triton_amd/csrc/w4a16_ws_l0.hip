// Instantiations of the LDS-staged-activation W4A16 kernel for the reference uint8 layout:
// token tiles of 1 .. 10 x 16 rows, BLOCK_N = 64 (RW 1) and 128 (RW 2).
#include "w4a16_tiles.hpp"

namespace specq {

const void* w4a16_ws_fn_l0(int mt, int rw) {
  switch (mt * 4 + rw) {
    case 5: return w4a16_ws_pick<1, 1, 0>();
    case 6: return w4a16_ws_pick<1, 2, 0>();
    case 9: return w4a16_ws_pick<2, 1, 0>();
    case 10: return w4a16_ws_pick<2, 2, 0>();
    case 13: return w4a16_ws_pick<3, 1, 0>();
    case 14: return w4a16_ws_pick<3, 2, 0>();
    case 17: return w4a16_ws_pick<4, 1, 0>();
    case 18: return w4a16_ws_pick<4, 2, 0>();
    case 21: return w4a16_ws_pick<5, 1, 0>();
    case 22: return w4a16_ws_pick<5, 2, 0>();
    case 25: return w4a16_ws_pick<6, 1, 0>();
    case 26: return w4a16_ws_pick<6, 2, 0>();
    case 29: return w4a16_ws_pick<7, 1, 0>();
    case 30: return w4a16_ws_pick<7, 2, 0>();
    case 33: return w4a16_ws_pick<8, 1, 0>();
    case 34: return w4a16_ws_pick<8, 2, 0>();
    case 37: return w4a16_ws_pick<9, 1, 0>();
    case 38: return w4a16_ws_pick<9, 2, 0>();
    case 41: return w4a16_ws_pick<10, 1, 0>();
    case 42: return w4a16_ws_pick<10, 2, 0>();
    default: return nullptr;
  }
}

}  // namespace specq
