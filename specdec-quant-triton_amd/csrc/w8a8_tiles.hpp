// Tile table of the W8A8 streaming kernels (rk: M <= 16 per chunk, direct activation loads;
// ws: LDS-staged activations), shared by the instantiation units and the C-ABI dispatcher.
//
// A channel width BLOCK_N maps to how the 4 waves of a workgroup split the work:
//   16  -> all 4 waves on the same 16 channels, each a quarter of the K steps (KW = 4)
//   32  -> 2 x 16 channels, K split 2 ways                                    (KW = 2)
//   64  -> 4 x 16 channels, the waves walk the same K steps                   (KW = 1)
//   128 -> 4 x 32 channels                                                     (KW = 1, RW = 2)
// A chunk of the ws kernel's activation ring covers 256 bytes of K (S K steps of each of the KW
// waves).  The ring holds 2 chunks, or 4 for the K-splitting tiles (16 and 32 channels) up to
// 96 token rows: measured on the Llama-3-8B linears, deeper rings only add queueing once a
// chunk carries 4 K steps per wave or the token tile is deep.
#pragma once
#include "w8a8_rk.hpp"
#include "w8a8_ws.hpp"

namespace specq {

constexpr int kW8A8MaxMt = 19;  // deepest token tile (304 rows)

template <int BNSEL>  // 0: 16, 1: 32, 2: 64, 3: 128 channels
struct W8A8BnSel {
  static constexpr int KW = BNSEL == 0 ? 4 : (BNSEL == 1 ? 2 : 1);
  static constexpr int RW = BNSEL == 3 ? 2 : 1;
  static constexpr int S = 4 / KW;  // K steps per wave per 256-byte chunk
};

// Ring slots of the ws kernel's activation chunks for a token depth and channel-block shape.
constexpr int w8a8_ws_nslot(int mt, int kw) { return (kw >= 2 && mt <= 6) ? 4 : 2; }

template <int MT, int BNSEL>
struct W8A8WsPick {
  using B = W8A8BnSel<BNSEL>;
  static constexpr int NSLOT = w8a8_ws_nslot(MT, B::KW);
  using Cfg = W8A8WsCfg<MT, B::RW, B::KW, B::S, NSLOT, 4>;
};

template <int MT, int BNSEL, int WL>
const void* w8a8_ws_pick() {
  using P = W8A8WsPick<MT, BNSEL>;
  using B = W8A8BnSel<BNSEL>;
  return reinterpret_cast<const void*>(&w8a8_ws_kernel<MT, B::RW, B::KW, B::S, P::NSLOT, 4, WL>);
}

template <int BNSEL, int WL>
const void* w8a8_rk_pick() {
  using B = W8A8BnSel<BNSEL>;
  return reinterpret_cast<const void*>(&w8a8_rk_kernel<1, B::RW, B::KW, 4, WL>);
}

// Defined in the instantiation units.
const void* w8a8_ws_fn_n16_l0(int mt);
const void* w8a8_ws_fn_n16_l1(int mt);
const void* w8a8_ws_fn_n32_l0(int mt);
const void* w8a8_ws_fn_n32_l1(int mt);
const void* w8a8_ws_fn_n64_l0(int mt);
const void* w8a8_ws_fn_n64_l1(int mt);
const void* w8a8_ws_fn_n128_l0(int mt);
const void* w8a8_ws_fn_n128_l1(int mt);
const void* w8a8_ws_fn_n16_l2(int mt);
const void* w8a8_ws_fn_n32_l2(int mt);
const void* w8a8_ws_fn_n64_l2(int mt);
const void* w8a8_ws_fn_n128_l2(int mt);
const void* w8a8_rk_fn(int bnsel, int layout);

}  // namespace specq
