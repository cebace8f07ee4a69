// Instantiations of the register-streaming W8A8 kernel, weight layout 0 (row-major), RW = 1.
#include "w8a8_stream.hpp"

namespace specq {

#define SPECQ_W8A8_STREAM_CASE(MT) \
  case MT: return reinterpret_cast<const void*>(&w8a8_stream_kernel<MT, 1, 0>);

const void* w8a8_stream_kernel_l0r1(int mt) {
  switch (mt) {
    SPECQ_W8A8_STREAM_CASE(1)
    SPECQ_W8A8_STREAM_CASE(2)
    SPECQ_W8A8_STREAM_CASE(3)
    SPECQ_W8A8_STREAM_CASE(4)
    SPECQ_W8A8_STREAM_CASE(5)
    SPECQ_W8A8_STREAM_CASE(6)
    SPECQ_W8A8_STREAM_CASE(7)
    SPECQ_W8A8_STREAM_CASE(8)
    SPECQ_W8A8_STREAM_CASE(9)
    SPECQ_W8A8_STREAM_CASE(10)
    SPECQ_W8A8_STREAM_CASE(11)
    SPECQ_W8A8_STREAM_CASE(12)
    SPECQ_W8A8_STREAM_CASE(13)
    SPECQ_W8A8_STREAM_CASE(14)
    SPECQ_W8A8_STREAM_CASE(15)
    SPECQ_W8A8_STREAM_CASE(16)
    SPECQ_W8A8_STREAM_CASE(17)
    SPECQ_W8A8_STREAM_CASE(18)
    SPECQ_W8A8_STREAM_CASE(19)
    SPECQ_W8A8_STREAM_CASE(20)
    default: return nullptr;
  }
}

}  // namespace specq
