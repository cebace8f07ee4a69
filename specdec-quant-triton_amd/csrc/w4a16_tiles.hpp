// Tile table of the W4A16 kernels, shared by the instantiation units and the C-ABI dispatcher.
//   rk (w4a16_rk.hpp): token tiles of 1-2 x 16 rows, activations loaded into registers.
//   ws (w4a16_ws.hpp): token tiles of 1-16 x 16 rows, activations staged in an LDS ring of
//      NSLOT chunks of S 128-wide K blocks (4 KB per block per 16 token rows), weights in a
//      register ring NSW blocks deep (W4WsPick).
// RW = 1 or 2 16-channel fragments per wave, i.e. BLOCK_N = 64 or 128 per workgroup.
#pragma once
#include "w4a16_rk.hpp"
#include "w4a16_ws.hpp"

namespace specq {

constexpr int kW4MaxMt = 16;    // deepest token tile (256 rows)
constexpr int kW4RkMaxMt = 2;

// LDS ring and weight-ring depth per tile (measured on the Llama-3-8B linears): chunks of 2
// blocks for 16-row tiles (1 beyond), 4 LDS slots up to 96 rows (2 beyond), and a weight ring
// as deep as the LDS ring but at least 4 blocks, as far as the wait counts fit the 6-bit load
// counter.  Deeper weight rings measured slower.
template <int MT, int RW, int LAYOUT>
struct W4WsPick {
  static constexpr int S = MT == 1 ? 2 : 1;
  static constexpr int WPER = RW * (1 + W4Nsc<LAYOUT>::value);
  static constexpr bool fits(int nslot, int nsw) {
    return (nsw - 1) * WPER + ((nsw - 1 + S - 1) / S) * MT * S <= 63 && (nslot - 1) * S * (WPER + MT) <= 63 &&
           nslot * MT * 16 * 256 * S <= 160 * 1024;
  }
  static constexpr int choose() {  // nslot * 100 + nsw
    for (int nslot = MT <= 6 ? 4 : 2; nslot >= 2; --nslot) {
      const int body = S * nslot;
      for (int nsw = ((4 + body - 1) / body) * body; nsw >= body; nsw -= body)
        if (fits(nslot, nsw)) return nslot * 100 + nsw;
    }
    return 0;
  }
  static constexpr int NSLOT = choose() / 100;
  static constexpr int NSW = choose() % 100;
  using Cfg = W4WsCfg<MT, RW, S, NSLOT, NSW, LAYOUT>;
};
// The same choice at run time (kernel names in resource queries).
int w4a16_ws_shape(int mt, int rw, int layout, int* s, int* nslot, int* nsw);

template <int MT, int RW, int LAYOUT>
const void* w4a16_ws_pick() {
  using P = W4WsPick<MT, RW, LAYOUT>;
  return reinterpret_cast<const void*>(&w4a16_ws_kernel<MT, RW, P::S, P::NSLOT, P::NSW, LAYOUT>);
}
template <int MT, int RW, int LAYOUT>
const void* w4a16_rk_pick() {
  return reinterpret_cast<const void*>(&w4a16_rk_kernel<MT, RW, LAYOUT>);
}

// Defined in the instantiation units.
const void* w4a16_ws_fn_l0(int mt, int rw);
const void* w4a16_ws_fn_l1(int mt, int rw);
const void* w4a16_ws_fn_l2(int mt, int rw);
const void* w4a16_rk_fn(int mt, int rw, int layout);

}  // namespace specq
