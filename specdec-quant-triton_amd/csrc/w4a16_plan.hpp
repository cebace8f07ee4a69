// Plan-mode W4A16 launch that holds several compiled tilings and picks one on the device.
//
// The W4A16 counterpart of w8a8_plan.hpp: a graph captured at the largest grid replays every
// active M = plan[0], and no single token-tile depth serves M = 1 and M = 288 alike.  This
// launch inlines a menu of the LDS-staged kernel's tilings (token-tile depth x 64 or 128
// channels per workgroup) and takes, per 16 rows of M, the tiling the eager cost model prices
// lowest at that step.  The split count, and with it the fp32 summation order, is a function
// of (N, K) only, the same for every entry, so every entry gives the bit-identical result of
// an eager call.
//
// Menu (index: token rows x channels): 0..1 16 x 64/128, 2..3 32, 4..5 48, 6..7 64, 8..9 80,
// 10 96 x 128, 11 112 x 128, 12..13 144.  Every tiling runs 8 waves in two streams, each with a
// 2-slot ring; the tilings share two slot variables of two stream halves each, sized for the
// largest tiling (4 x 144 rows x 256 bytes, 144 KB).
#pragma once
#include "w4a16_tiles.hpp"

namespace specq {

constexpr int kW4PlanRows = 19;  // entries: M in (16 e, 16 (e + 1)]; the last also beyond
constexpr int kW4PlanMenu = 14;
constexpr int kW4PlanMenuMt[kW4PlanMenu] = {1, 1, 2, 2, 3, 3, 4, 4, 5, 5, 6, 7, 9, 9};
constexpr int kW4PlanMenuRw[kW4PlanMenu] = {1, 2, 1, 2, 1, 2, 1, 2, 1, 2, 2, 2, 1, 2};
constexpr int kW4PlanSlotA = 9 * 16 * 256;  // slots 0, 1
constexpr int kW4PlanSlotB = 16;            // slots 2, 3 (unused by 2-slot rings)

struct W4PlanTile {
  int path;  // menu index
  int n_tiles, m_chunks;
};
struct W4PlanParams {
  W4A16Params p;
  W4PlanTile t[kW4PlanRows];
};

template <int I, int LAYOUT, class SlotPtr>
__device__ __forceinline__ void w4a16_plan_path(const W4A16Params& p, SlotPtr slots) {
  constexpr int MT = kW4PlanMenuMt[I], RW = kW4PlanMenuRw[I];
  using P = W4WsPick<MT, RW, LAYOUT>;
  static_assert(P::Cfg::SLOT <= kW4PlanSlotA && (P::NSLOT <= 2 || P::Cfg::SLOT <= kW4PlanSlotB) && P::NSLOT <= 4 &&
                    4 * RW * MT * 1024 <= 2 * kW4PlanSlotA,
                "menu tiling fits the shared slots");
  w4a16_ws_body<MT, RW, P::S, P::NSLOT, P::NSW, LAYOUT>(p, slots);
}

template <int LAYOUT>
__global__ __launch_bounds__(kW4WsThreads) void w4a16_plan_kernel(W4PlanParams pp) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_s0[2][kW4PlanSlotA], lds_s1[2][kW4PlanSlotA];
  __shared__ __attribute__((aligned(16))) uint8_t lds_s2[2][kW4PlanSlotB], lds_s3[2][kW4PlanSlotB];
  auto slots = [&](auto ic, int h) -> uint8_t* {
    constexpr int i = decltype(ic)::value;
    static_assert(i < 4, "menu tilings use at most four slots");
    if constexpr (i == 0) return lds_s0[h];
    else if constexpr (i == 1) return lds_s1[h];
    else if constexpr (i == 2) return lds_s2[h];
    else return lds_s3[h];
  };
  int M = min(max(pp.p.plan[0], 0), pp.p.m_grid);
  M = uniform(M);
  const int e = uniform(min(max((M + 15) / 16, 1), kW4PlanRows) - 1);
  W4A16Params p = pp.p;
  const W4PlanTile& t = pp.t[e];
  p.n_tiles = t.n_tiles; p.m_chunks = t.m_chunks; p.units = t.n_tiles * p.splits;
  switch (uniform(t.path)) {
    case 0: w4a16_plan_path<0, LAYOUT>(p, slots); break;
    case 1: w4a16_plan_path<1, LAYOUT>(p, slots); break;
    case 2: w4a16_plan_path<2, LAYOUT>(p, slots); break;
    case 3: w4a16_plan_path<3, LAYOUT>(p, slots); break;
    case 4: w4a16_plan_path<4, LAYOUT>(p, slots); break;
    case 5: w4a16_plan_path<5, LAYOUT>(p, slots); break;
    case 6: w4a16_plan_path<6, LAYOUT>(p, slots); break;
    case 7: w4a16_plan_path<7, LAYOUT>(p, slots); break;
    case 8: w4a16_plan_path<8, LAYOUT>(p, slots); break;
    case 9: w4a16_plan_path<9, LAYOUT>(p, slots); break;
    case 10: w4a16_plan_path<10, LAYOUT>(p, slots); break;
    case 11: w4a16_plan_path<11, LAYOUT>(p, slots); break;
    case 12: w4a16_plan_path<12, LAYOUT>(p, slots); break;
    case 13: w4a16_plan_path<13, LAYOUT>(p, slots); break;
    default: break;
  }
}

}  // namespace specq
