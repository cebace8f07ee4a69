// Instantiations of the LDS-DMA W8A8 kernel with RW = 2, NWN = 2 (BLOCK_N = 64).
// BLOCK_M = 16..240: deeper tiles would not fit two ring slots of 256-byte K blocks in LDS.
#include "w8a8_dma.hpp"

namespace specq {

#define SPECQ_W8A8_DMA_CASE(MT) \
  case MT: return reinterpret_cast<const void*>(&w8a8_dma_kernel<MT, 2, 2>);

const void* w8a8_dma_kernel_r2n2(int mt) {
  switch (mt) {
    SPECQ_W8A8_DMA_CASE(1)
    SPECQ_W8A8_DMA_CASE(2)
    SPECQ_W8A8_DMA_CASE(3)
    SPECQ_W8A8_DMA_CASE(4)
    SPECQ_W8A8_DMA_CASE(5)
    SPECQ_W8A8_DMA_CASE(6)
    SPECQ_W8A8_DMA_CASE(7)
    SPECQ_W8A8_DMA_CASE(8)
    SPECQ_W8A8_DMA_CASE(9)
    SPECQ_W8A8_DMA_CASE(10)
    SPECQ_W8A8_DMA_CASE(11)
    SPECQ_W8A8_DMA_CASE(12)
    SPECQ_W8A8_DMA_CASE(13)
    SPECQ_W8A8_DMA_CASE(14)
    SPECQ_W8A8_DMA_CASE(15)
    default: return nullptr;
  }
}

int w8a8_dma_lds_r2n2(int mt) {
  switch (mt) {
    case 1: return W8A8DmaCfg<1, 2, 2>::LDS_BYTES;
    case 2: return W8A8DmaCfg<2, 2, 2>::LDS_BYTES;
    case 3: return W8A8DmaCfg<3, 2, 2>::LDS_BYTES;
    case 4: return W8A8DmaCfg<4, 2, 2>::LDS_BYTES;
    case 5: return W8A8DmaCfg<5, 2, 2>::LDS_BYTES;
    case 6: return W8A8DmaCfg<6, 2, 2>::LDS_BYTES;
    case 7: return W8A8DmaCfg<7, 2, 2>::LDS_BYTES;
    case 8: return W8A8DmaCfg<8, 2, 2>::LDS_BYTES;
    case 9: return W8A8DmaCfg<9, 2, 2>::LDS_BYTES;
    case 10: return W8A8DmaCfg<10, 2, 2>::LDS_BYTES;
    case 11: return W8A8DmaCfg<11, 2, 2>::LDS_BYTES;
    case 12: return W8A8DmaCfg<12, 2, 2>::LDS_BYTES;
    case 13: return W8A8DmaCfg<13, 2, 2>::LDS_BYTES;
    case 14: return W8A8DmaCfg<14, 2, 2>::LDS_BYTES;
    case 15: return W8A8DmaCfg<15, 2, 2>::LDS_BYTES;
    default: return -1;
  }
}

}  // namespace specq
