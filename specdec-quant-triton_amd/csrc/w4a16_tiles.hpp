// Tile table of the W4A16 kernels, shared by the instantiation units and the C-ABI dispatcher.
//   rk (w4a16_rk.hpp): token tiles of 1-2 x 16 rows, activations loaded into registers.
//   ws (w4a16_ws.hpp): token tiles of 1-10 x 16 rows, 8 waves in two K streams, each stream's
//      activations staged in an LDS ring of NSLOT chunks of S 128-wide K blocks (4 KB per
//      block per 16 token rows), weights in a register ring NSW blocks deep (W4WsPick).
// RW = 1 or 2 16-channel fragments per wave, i.e. BLOCK_N = 64 or 128 per workgroup.
#pragma once
#include "w4a16_rk.hpp"
#include "w4a16_ws.hpp"

namespace specq {

constexpr int kW4MaxMt = 10;    // deepest token tile (160 rows: two streams x two 40 KB LDS slots = 160 KB)
constexpr int kW4RkMaxMt = 2;

// LDS ring and weight-ring depth per tile (measured on the Llama-3-8B linears, 8-wave
// kernel): chunks of 2 blocks for 16-row tiles (1 beyond), 2 LDS slots per stream (one chunk
// in flight ahead of the one being multiplied), and a weight ring as deep as the LDS ring (2
// blocks per stream, 4 for 16-row tiles); deeper rings of either kind measured slower.
template <int MT, int RW, int LAYOUT>
struct W4WsPick {
  static constexpr int S = MT == 1 ? 2 : 1;
  static constexpr int NSLOT = 2;
  static constexpr int NSW = S * NSLOT;
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
