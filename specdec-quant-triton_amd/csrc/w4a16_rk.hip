// Instantiations of the register-stream W4A16 kernel: token tiles of 1 and 2 x 16 rows,
// BLOCK_N = 64 (RW 1) and 128 (RW 2), all three weight layouts; and the run-time view of the
// LDS-staged kernel's ring shapes.
#include "w4a16_tiles.hpp"

namespace specq {

template <int LAYOUT>
static const void* rk_for_layout(int mt, int rw) {
  switch (mt * 4 + rw) {
    case 5: return w4a16_rk_pick<1, 1, LAYOUT>();
    case 6: return w4a16_rk_pick<1, 2, LAYOUT>();
    case 9: return w4a16_rk_pick<2, 1, LAYOUT>();
    case 10: return w4a16_rk_pick<2, 2, LAYOUT>();
    default: return nullptr;
  }
}

template <int MT, int RW, int LAYOUT>
static int shape_of(int* s, int* nslot, int* nsw) {
  using P = W4WsPick<MT, RW, LAYOUT>;
  *s = P::S; *nslot = P::NSLOT; *nsw = P::NSW;
  return 0;
}

template <int MT>
static int shape_mt(int rw, int layout, int* s, int* nslot, int* nsw) {
  switch (rw * 4 + layout) {
    case 4: return shape_of<MT, 1, 0>(s, nslot, nsw);
    case 5: return shape_of<MT, 1, 1>(s, nslot, nsw);
    case 6: return shape_of<MT, 1, 2>(s, nslot, nsw);
    case 8: return shape_of<MT, 2, 0>(s, nslot, nsw);
    case 9: return shape_of<MT, 2, 1>(s, nslot, nsw);
    case 10: return shape_of<MT, 2, 2>(s, nslot, nsw);
  }
  return -1;
}

template <int MT>
static int shape_find(int mt, int rw, int layout, int* s, int* nslot, int* nsw) {
  if (mt == MT) return shape_mt<MT>(rw, layout, s, nslot, nsw);
  if constexpr (MT < kW4MaxMt) return shape_find<MT + 1>(mt, rw, layout, s, nslot, nsw);
  return -1;
}

int w4a16_ws_shape(int mt, int rw, int layout, int* s, int* nslot, int* nsw) {
  return shape_find<1>(mt, rw, layout, s, nslot, nsw);
}

const void* w4a16_rk_fn(int mt, int rw, int layout) {
  switch (layout) {
    case 0: return rk_for_layout<0>(mt, rw);
    case 1: return rk_for_layout<1>(mt, rw);
    case 2: return rk_for_layout<2>(mt, rw);
    default: return nullptr;
  }
}

}  // namespace specq
