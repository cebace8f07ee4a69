// Instantiations of the W4A16 kernel for packed layout 0: MT = 1..16 token blocks
// (BLOCK_M = 16*MT) and RW = 1 or 2 sixteen-channel fragments per wave.
#include "w4a16.hpp"

namespace specq {

#define SPECQ_W4_CASE(MT, RW) \
  case MT * 4 + RW: return reinterpret_cast<const void*>(&w4a16_kernel<MT, RW, 0>);

const void* w4a16_kernel_l0(int mt, int rw) {
  switch (mt * 4 + rw) {
    SPECQ_W4_CASE(1, 1)
    SPECQ_W4_CASE(1, 2)
    SPECQ_W4_CASE(2, 1)
    SPECQ_W4_CASE(2, 2)
    SPECQ_W4_CASE(3, 1)
    SPECQ_W4_CASE(3, 2)
    SPECQ_W4_CASE(4, 1)
    SPECQ_W4_CASE(4, 2)
    SPECQ_W4_CASE(5, 1)
    SPECQ_W4_CASE(5, 2)
    SPECQ_W4_CASE(6, 1)
    SPECQ_W4_CASE(6, 2)
    SPECQ_W4_CASE(7, 1)
    SPECQ_W4_CASE(7, 2)
    SPECQ_W4_CASE(8, 1)
    SPECQ_W4_CASE(8, 2)
    SPECQ_W4_CASE(9, 1)
    SPECQ_W4_CASE(9, 2)
    SPECQ_W4_CASE(10, 1)
    SPECQ_W4_CASE(10, 2)
    SPECQ_W4_CASE(11, 1)
    SPECQ_W4_CASE(11, 2)
    SPECQ_W4_CASE(12, 1)
    SPECQ_W4_CASE(12, 2)
    SPECQ_W4_CASE(13, 1)
    SPECQ_W4_CASE(13, 2)
    SPECQ_W4_CASE(14, 1)
    SPECQ_W4_CASE(14, 2)
    SPECQ_W4_CASE(15, 1)
    SPECQ_W4_CASE(15, 2)
    SPECQ_W4_CASE(16, 1)
    SPECQ_W4_CASE(16, 2)
    default: return nullptr;
  }
}

}  // namespace specq
