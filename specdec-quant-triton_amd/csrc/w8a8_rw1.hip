// Instantiations of the W8A8 kernel for 1 x 16 output channels per workgroup.
// Every M-tile size MT = 1..20 (BLOCK_M = 16*MT) is built for 16-byte aligned operands;
// the sub-16-byte alignments (odd K or strides) get the BLOCK_M values 16/32/64/128/256/320.
#include "w8a8.hpp"

namespace specq {

#define SPECQ_W8A8_CASE(MT, VEC) \
  case MT * 32 + VEC: return reinterpret_cast<const void*>(&w8a8_kernel<MT, 1, VEC>);

const void* w8a8_kernel_rw1(int mt, int vec) {
  switch (mt * 32 + vec) {
    SPECQ_W8A8_CASE(1, 16)
    SPECQ_W8A8_CASE(2, 16)
    SPECQ_W8A8_CASE(3, 16)
    SPECQ_W8A8_CASE(4, 16)
    SPECQ_W8A8_CASE(5, 16)
    SPECQ_W8A8_CASE(6, 16)
    SPECQ_W8A8_CASE(7, 16)
    SPECQ_W8A8_CASE(8, 16)
    SPECQ_W8A8_CASE(9, 16)
    SPECQ_W8A8_CASE(10, 16)
    SPECQ_W8A8_CASE(11, 16)
    SPECQ_W8A8_CASE(12, 16)
    SPECQ_W8A8_CASE(13, 16)
    SPECQ_W8A8_CASE(14, 16)
    SPECQ_W8A8_CASE(15, 16)
    SPECQ_W8A8_CASE(16, 16)
    SPECQ_W8A8_CASE(17, 16)
    SPECQ_W8A8_CASE(18, 16)
    SPECQ_W8A8_CASE(19, 16)
    SPECQ_W8A8_CASE(20, 16)
    SPECQ_W8A8_CASE(1, 8)
    SPECQ_W8A8_CASE(1, 4)
    SPECQ_W8A8_CASE(1, 1)
    SPECQ_W8A8_CASE(2, 8)
    SPECQ_W8A8_CASE(2, 4)
    SPECQ_W8A8_CASE(2, 1)
    SPECQ_W8A8_CASE(4, 8)
    SPECQ_W8A8_CASE(4, 4)
    SPECQ_W8A8_CASE(4, 1)
    SPECQ_W8A8_CASE(8, 8)
    SPECQ_W8A8_CASE(8, 4)
    SPECQ_W8A8_CASE(8, 1)
    SPECQ_W8A8_CASE(16, 8)
    SPECQ_W8A8_CASE(16, 4)
    SPECQ_W8A8_CASE(16, 1)
    SPECQ_W8A8_CASE(20, 8)
    SPECQ_W8A8_CASE(20, 4)
    SPECQ_W8A8_CASE(20, 1)
    default: return nullptr;
  }
}

}  // namespace specq
