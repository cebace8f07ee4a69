// W4A16 GEMM, register K-stream schedule (16- and 32-row token tiles): weights, scales and
// activations go straight from memory into MFMA operand registers; no LDS on the main loop.
//
// Arithmetic and fp32 summation order: w4a16.hpp (reference kernels.py:94-135).
//
//  * 4 waves per workgroup, each owning RW 16-channel fragments of the workgroup's BN = 64*RW
//    channels and all MT token tiles.  Per 128-wide K block a lane issues RW 16-byte weight
//    loads, RW (two for the reference layout) 4-byte scale loads and 4*MT 16-byte activation
//    loads; the 4 waves read the same activation bytes at about the same time, so all but the
//    first find them in the L1.  Each weight fragment is dequantized once and feeds MT MFMAs.
//  * Loads run NS-1 blocks ahead through a register ring.  Every loop iteration issues the same
//    loads (blocks past the split's range are out-of-range buffer reads that return zero and
//    add nothing), so a compile-time s_waitcnt vmcnt separates the block being multiplied
//    from the blocks in flight.
//  * The workgroup's K range is its split (contiguous blocks).  The blocks at even and odd
//    local index are summed into two accumulator sets (the two streams of the summation order,
//    w4a16.hpp), added as even + odd at the end; splits are summed in order by the last
//    workgroup to arrive (w4_splitk_finish).
#pragma once
#include "w4a16.hpp"

namespace specq {

template <int MT, int RW, int LAYOUT>
struct W4RkCfg {
  static constexpr int NSC = W4Nsc<LAYOUT>::value;
  static constexpr int BM = MT * 16, BNW = RW * 16, BN = 4 * BNW;
  static constexpr int PER = RW * (1 + NSC) + 4 * MT;   // loads per block per wave
  static constexpr int VG = RW * (4 + NSC) + 16 * MT;   // VGPRs per ring slot
  static constexpr int NS_REG = 168 / VG, NS_CNT = 63 / PER;
  static constexpr int NS0 = NS_REG < NS_CNT ? NS_REG : NS_CNT;
  // Even, so a block's parity within the split is its ring slot's (see the accumulators).
  static constexpr int NS = NS0 > 8 ? 8 : (NS0 < 2 ? 2 : (NS0 & ~1));
  static constexpr int D = NS - 1;
  static constexpr bool OK = D * PER <= 63;
};

template <int MT, int RW, int LAYOUT>
__global__ __launch_bounds__(256) void w4a16_rk_kernel(W4A16Params p) {
  using C = W4RkCfg<MT, RW, LAYOUT>;
  static_assert(C::OK, "W4A16 register-stream tile does not fit the load counter");
  constexpr int BM = C::BM, BNW = C::BNW, BN = C::BN, NS = C::NS, D = C::D, PER = C::PER, NSC = C::NSC;
  tl_mark(p.tl, p.tl_cap, 0);  // diagnostics build: workgroup start

  int mc, tile, split;
  if (!w4_decode_id(p, mc, tile, split)) return;
  int M = p.M;
  if (p.plan != nullptr) M = min(max(p.plan[0], 0), p.m_grid);
  M = uniform(M);
  const int m0 = mc * BM;
  if (m0 >= M) return;

  const int lane = lane_id(), w = uniform(wave_id()), g = lane >> 4, r = lane & 15;
  const int ltile = w4_select_member(p, tile);  // tile within its GEMM (weights, outputs)
  const int n0 = ltile * BN + w * BNW;  // first channel of this wave
  const int blk0 = split * p.bps;
  const int cnt = max(0, min(p.nblocks, blk0 + p.bps) - blk0);
  const int halfK = p.K / 2;

  W4Weights<RW, LAYOUT> wt;
  wt.init(p, n0);
  const int m_rows = min(BM, M - m0);
  const rsrc_t asrc = make_rsrc(p.A + (int64_t)m0 * p.lda, (uint32_t)(((m_rows - 1) * p.lda + p.K) * 2));
  uint32_t arow[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) arow[j] = (16 * j + r < m_rows) ? (uint32_t)((16 * j + r) * p.lda * 2) : kOOB;

  // Per-lane copy of the loop bound: a wave-uniform bound turns the load masks into branches,
  // and a branch around a load costs a full vmcnt wait at the join.
  int cnt_v = cnt;
  asm volatile("" : "+v"(cnt_v));

  auto issue = [&](int i, v4i (&wv)[RW], uint32_t (&sv)[RW][NSC], v4i (&av)[MT][4]) {
    const int b = blk0 + i;
    const bool live = i < cnt_v;
    wt.issue(b, live, wv, sv);
#pragma unroll
    for (int j = 0; j < MT; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u)
        av[j][u] = __builtin_amdgcn_raw_buffer_load_b128(
            asrc, oob_unless(live & (arow[j] != kOOB), arow[j] + (uint32_t)(2 * w4_k<LAYOUT>(b, u, g, halfK))), 0, 0);
  };

  v4f acc[2][RW][MT];  // [stream: local block parity]
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j) acc[h][i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  v4i wring[NS][RW];
  uint32_t sring[NS][RW][NSC];
  v4i aring[NS][MT][4];
  // Prologue: blocks 0 .. D-1 in flight, in block order (the scheduling barriers keep the
  // load order identical to the loop's, so the compiler's wait counts agree on both paths).
  static_for<0, D>([&](auto sc) {
    constexpr int s = decltype(sc)::value;
    issue(s, wring[s], sring[s], aring[s]);
    __builtin_amdgcn_sched_barrier(0);
  });
  const int turns = (cnt + NS - 1) / NS;
  for (int it = 0; it < turns; ++it) {
    static_for<0, NS>([&](auto tc) __attribute__((always_inline)) {
      constexpr int t = decltype(tc)::value;
      constexpr int tn = (t + D) % NS;
      issue(it * NS + t + D, wring[tn], sring[tn], aring[tn]);
      __builtin_amdgcn_sched_barrier(0);
      wait_vmcnt<D * PER>();
      const int b = blk0 + it * NS + t;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        v8h wf[RW];
#pragma unroll
        for (int i = 0; i < RW; ++i) wf[i] = wt.frag(b, i, u, wring[t], sring[t]);
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          const v8h af = __builtin_bit_cast(v8h, aring[t][j][u]);
#pragma unroll
          for (int i = 0; i < RW; ++i) acc[t & 1][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[i], af, acc[t & 1][i][j], 0, 0, 0);
        }
      }
    });
  }
  wait_vmcnt<0>();
  tl_mark(p.tl, p.tl_cap, 2);  // diagnostics build: main loop done
  v4f sum[RW][MT];
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) sum[i][j] = acc[0][i][j] + acc[1][i][j];

  __shared__ int s_last_rk4;
  w4_epilogue<MT, RW, BM, BN>(p, sum, mc, tile, split, m0, n0, w * BNW, M, &s_last_rk4);
}

}  // namespace specq
