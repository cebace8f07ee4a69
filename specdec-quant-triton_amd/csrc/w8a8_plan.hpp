// Plan-mode W8A8 launch that holds several compiled tilings and picks one on the device.
//
// A graph captured at the largest grid replays every active M = plan[0].  No single token-tile
// depth serves M = 1 and M = 288 alike (a 16-row direct-activation tile is fastest at decode,
// 144-row tiles at the top of the range), and a streaming kernel's per-chunk costs are fixed
// by its compiled depth.  So this launch inlines a menu of the library's own tilings (the RK and
// WS kernel bodies) and takes, per 16 rows of M, a tiling chosen on the host by the same cost
// model as eager calls: workgroup w reads M, looks up the entry of ceil(M / 16) in the
// parameter block, and runs that tiling's body with that entry's channel tiles, M-chunks and
// split count (workgroups past the tiling's own grid exit at once).  INT32 sums are exact, so
// every entry gives the bit-identical result of an eager call.
//
// Two menus (index: token-tile depth x channel block), one launch variant each:
//   variant 0                                   variant 1 (deep tiles, 2-slot rings only)
//   0..3   16-row direct tile, 16/32/64/128     0..3   16-row direct tile, 16/32/64/128
//   4..7   32-row, 16/32/64/128                 4..5   32-row, 64/128
//   8..10  48-row, 32/64/128                    6..7   48-row, 64/128
//   11..12 64-row, 64/128                       8..9   64-row, 64/128
//   13..15 80-row, 32/64/128                    10..11 80-row, 64/128
//   16..17 144-row, 64/128                      12..13 144-row, 64/128
//                                               14     160-row, 128
//                                               15..16 192-row, 64/128
//                                               17     224-row, 128
//                                               18     256-row, 128
//                                               19..20 288-row, 64/128
// The streaming tilings of a variant share four LDS slots sized for its largest tiling:
// variant 0 two of 144 rows x 256 bytes and two of 80 x 256 (the 4-slot rings of the
// K-splitting tiles), 112 KB; variant 1 two of 288 x 256, 144 KB.  The host takes the variant
// whose table the cost model prices lower over the steps of M (the deep one for wide GEMMs
// such as gate|up, whose large-M steps want one chunk of all rows).
#pragma once
#include "w8a8_tiles.hpp"

namespace specq {

constexpr int kW8A8PlanRows = 19;   // entries: M in (16 e, 16 (e + 1)]; the last also beyond
constexpr int kW8A8PlanMenu = 21;  // entries of the longer menu; variant 0 repeats its last
// (token tiles of 16 rows, channel-width selector) of each menu entry; depth 1 = direct-activation.
constexpr int kW8A8PlanMenuMt[2][kW8A8PlanMenu] = {
    {1, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 4, 4, 5, 5, 5, 9, 9, 9, 9, 9},
    {1, 1, 1, 1, 2, 2, 3, 3, 4, 4, 5, 5, 9, 9, 10, 12, 12, 14, 16, 18, 18}};
constexpr int kW8A8PlanMenuSel[2][kW8A8PlanMenu] = {
    {0, 1, 2, 3, 0, 1, 2, 3, 1, 2, 3, 2, 3, 1, 2, 3, 2, 3, 3, 3, 3},
    {0, 1, 2, 3, 2, 3, 2, 3, 2, 3, 2, 3, 2, 3, 3, 2, 3, 3, 3, 2, 3}};
constexpr int kW8A8PlanSlotA[2] = {9 * 16 * 256, 18 * 16 * 256};  // slots 0, 1
constexpr int kW8A8PlanSlotB[2] = {5 * 16 * 256, 16};             // slots 2, 3

struct W8A8PlanTile {
  int path;                           // menu index
  int n_tiles, m_chunks, splits, k_range;
  int grp_tile_end[3];                // grouped launches: member boundaries in this tiling's tiles
};
struct W8A8PlanParams {
  W8A8Params p;
  W8A8PlanTile t[kW8A8PlanRows];
};

template <int I, int WL, int V, class SlotPtr>
__device__ __forceinline__ void w8a8_plan_path(const W8A8Params& p, SlotPtr slots) {
  constexpr int MT = kW8A8PlanMenuMt[V][I], SEL = kW8A8PlanMenuSel[V][I];
  using B = W8A8BnSel<SEL>;
  if constexpr (MT == 1) {
    w8a8_rk_body<1, B::RW, B::KW, 4, WL>(p);
  } else {
    using P = W8A8WsPick<MT, SEL>;
    static_assert(P::Cfg::SLOT <= kW8A8PlanSlotA[V] && (P::NSLOT <= 2 || P::Cfg::SLOT <= kW8A8PlanSlotB[V]),
                  "menu tiling fits the shared slots");
    w8a8_ws_body<MT, B::RW, B::KW, B::S, P::NSLOT, 4, WL>(p, slots);
  }
}

template <int WL, int V>
__global__ __launch_bounds__(256) void w8a8_plan_kernel(W8A8PlanParams pp) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_s0[kW8A8PlanSlotA[V]], lds_s1[kW8A8PlanSlotA[V]];
  __shared__ __attribute__((aligned(16))) uint8_t lds_s2[kW8A8PlanSlotB[V]], lds_s3[kW8A8PlanSlotB[V]];
  auto slots = [&](auto ic) -> uint8_t* {
    constexpr int i = decltype(ic)::value;
    static_assert(i < 4, "menu tilings use at most four slots");
    if constexpr (i == 0) return lds_s0;
    else if constexpr (i == 1) return lds_s1;
    else if constexpr (i == 2) return lds_s2;
    else return lds_s3;
  };
  int M = min(max(pp.p.plan[0], 0), pp.p.m_grid);
  M = uniform(M);
  const int e = uniform(min(max((M + 15) / 16, 1), kW8A8PlanRows) - 1);
  W8A8Params p = pp.p;
  const W8A8PlanTile& t = pp.t[e];
  p.n_tiles = t.n_tiles; p.m_chunks = t.m_chunks; p.splits = t.splits; p.k_range = t.k_range;
  p.grp_tile_end[0] = t.grp_tile_end[0]; p.grp_tile_end[1] = t.grp_tile_end[1]; p.grp_tile_end[2] = t.grp_tile_end[2];
  switch (uniform(t.path)) {
    case 0: w8a8_plan_path<0, WL, V>(p, slots); break;
    case 1: w8a8_plan_path<1, WL, V>(p, slots); break;
    case 2: w8a8_plan_path<2, WL, V>(p, slots); break;
    case 3: w8a8_plan_path<3, WL, V>(p, slots); break;
    case 4: w8a8_plan_path<4, WL, V>(p, slots); break;
    case 5: w8a8_plan_path<5, WL, V>(p, slots); break;
    case 6: w8a8_plan_path<6, WL, V>(p, slots); break;
    case 7: w8a8_plan_path<7, WL, V>(p, slots); break;
    case 8: w8a8_plan_path<8, WL, V>(p, slots); break;
    case 9: w8a8_plan_path<9, WL, V>(p, slots); break;
    case 10: w8a8_plan_path<10, WL, V>(p, slots); break;
    case 11: w8a8_plan_path<11, WL, V>(p, slots); break;
    case 12: w8a8_plan_path<12, WL, V>(p, slots); break;
    case 13: w8a8_plan_path<13, WL, V>(p, slots); break;
    case 14: w8a8_plan_path<14, WL, V>(p, slots); break;
    case 15: w8a8_plan_path<15, WL, V>(p, slots); break;
    case 16: w8a8_plan_path<16, WL, V>(p, slots); break;
    case 17: w8a8_plan_path<17, WL, V>(p, slots); break;
    case 18: w8a8_plan_path<18, WL, V>(p, slots); break;
    case 19: w8a8_plan_path<19, WL, V>(p, slots); break;
    case 20: w8a8_plan_path<20, WL, V>(p, slots); break;
    default: break;
  }
}

}  // namespace specq
