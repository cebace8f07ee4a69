// Instantiations of the LDS-shared-activation streaming W8A8 kernel, weight layout 0
// (row-major), RW = 2.  Tiles without room for a block in flight return null.
#include "w8a8_stream2.hpp"

namespace specq {

template <int MT>
static const void* stream2_pick(int* lds) {
  using C = W8A8Stream2Cfg<MT, 2, 0>;
  if constexpr (C::OK) {
    *lds = C::LDS_BYTES;
    return reinterpret_cast<const void*>(&w8a8_stream2_kernel<MT, 2, 0>);
  } else {
    return nullptr;
  }
}

#define SPECQ_W8A8_STREAM2_CASE(MT) \
  case MT: return stream2_pick<MT>(lds);

const void* w8a8_stream2_kernel_l0r2(int mt, int* lds) {
  switch (mt) {
    SPECQ_W8A8_STREAM2_CASE(1)
    SPECQ_W8A8_STREAM2_CASE(2)
    SPECQ_W8A8_STREAM2_CASE(3)
    SPECQ_W8A8_STREAM2_CASE(4)
    SPECQ_W8A8_STREAM2_CASE(5)
    SPECQ_W8A8_STREAM2_CASE(6)
    SPECQ_W8A8_STREAM2_CASE(7)
    SPECQ_W8A8_STREAM2_CASE(8)
    SPECQ_W8A8_STREAM2_CASE(9)
    SPECQ_W8A8_STREAM2_CASE(10)
    SPECQ_W8A8_STREAM2_CASE(11)
    SPECQ_W8A8_STREAM2_CASE(12)
    SPECQ_W8A8_STREAM2_CASE(13)
    SPECQ_W8A8_STREAM2_CASE(14)
    SPECQ_W8A8_STREAM2_CASE(15)
    SPECQ_W8A8_STREAM2_CASE(16)
    SPECQ_W8A8_STREAM2_CASE(17)
    SPECQ_W8A8_STREAM2_CASE(18)
    SPECQ_W8A8_STREAM2_CASE(19)
    SPECQ_W8A8_STREAM2_CASE(20)
    default: return nullptr;
  }
}

}  // namespace specq
