// W8A8 GEMM, register K-stream schedule: every operand goes straight from memory into MFMA
// operand registers, with no LDS staging on the main loop.
//
// Same arithmetic as w8a8_kernel (reference kernels.py:27-55): INT8 x INT8 products summed
// exactly in INT32, then (acc * sa[m]) * sw[n] in fp32 and one RNE cast to fp16.
//
// Schedule (NW 64-wide waves per workgroup):
//  * The weight is the MFMA A operand.  Each load instruction fetches one 16-row x 64-byte
//    MFMA fragment: lane l reads 16 bytes of row (l % 16) at K offset 16 * (l / 16) of the
//    64-byte K step (row-major weight), or one contiguous 1 KB pre-packed fragment (LAYOUT 1,
//    fragments stored K-step-major so concurrently running workgroups read adjacent memory).
//    The activations are the B operand, fetched the same way from the L2-resident activation
//    rows.  Both land in the registers the MFMA reads, so the main loop is loads + MFMAs only.
//  * A wave owns RW 16-channel tiles and MT 16-token tiles and keeps their INT32 sums in
//    registers for its whole K range: each activation fragment feeds RW MFMAs and each
//    weight fragment MT MFMAs.  The NW waves of a workgroup are KW waves along K (interleaved
//    64-byte steps, reduced through LDS at the end) times NW/KW waves along channels (which
//    read the same activation bytes at the same time, so all but the first hit the L1).
//  * Loads run NS-1 K steps ahead of the MFMAs through a register ring of NS slots.  Every
//    iteration issues the same number of loads (out-of-range ones are turned into buffer
//    reads past the descriptor's range, which return zero), so a compile-time s_waitcnt
//    vmcnt separates the step being multiplied from the steps in flight.
//  * With the row-major weight, workgroups start their K walk at staggered offsets (the
//    order of INT32 additions does not change the sum), so the workgroups running at one
//    time read different column ranges of the weight rows instead of all hitting the same
//    HBM channels.
//  * Split-K across workgroups hands INT32 tiles off 16 bytes per lane (w8a8_splitk_finish);
//    plan mode and the epilogue are shared with w8a8_kernel.
//  * Used for short token batches (M <= 16): one activation fragment per K step is cheap to
//    fetch per wave, and without LDS staging any number of waves can split K.
//  * LAYOUT 2 is the packed INT4 weight of W4A8 (w8a8_wop): half the weight bytes per step,
//    INT32 sums shifted right by 4 (exact) before the shared epilogue.
#pragma once
#include "w8a8.hpp"

namespace specq {

template <int MT, int RW, int KW, int NW>
struct W8A8RkCfg {
  static constexpr int CW = NW / KW;                    // waves along channels
  static constexpr int BM = MT * 16, BNW = RW * 16, BN = CW * BNW;
  static constexpr int PER = RW + MT;                   // loads per K step per wave
  // Ring depth: at most ~128 VGPRs of operands in flight and 63 outstanding loads.
  static constexpr int NS_REG = 128 / (4 * PER);
  static constexpr int NS_CNT = 63 / PER;
  static constexpr int NS0 = NS_REG < NS_CNT ? NS_REG : NS_CNT;
  static constexpr int NS = NS0 > 8 ? 8 : (NS0 < 2 ? 2 : NS0);
  static constexpr int D = NS - 1;                      // steps in flight
  static constexpr int RED_BYTES = (KW - 1) * BM * BN * 4;     // one slice per non-owner wave
};

// The kernel body, also inlined into the plan-mode launch that holds several tilings
// (w8a8_plan.hpp).
template <int MT, int RW, int KW, int NW, int LAYOUT>
__device__ __forceinline__ void w8a8_rk_body(W8A8Params p) {
  using C = W8A8RkCfg<MT, RW, KW, NW>;
  constexpr int CW = C::CW, BM = C::BM, BNW = C::BNW, BN = C::BN, NS = C::NS, D = C::D, PER = C::PER;
  extern __shared__ __attribute__((aligned(16))) int32_t smem_rk[];
  tl_mark(p.tl, p.tl_cap, 0);  // diagnostics build: workgroup start

  int mc, unit;
  if (!chunked_unit(p.m_chunks, p.n_tiles * p.splits, mc, unit)) return;
  int split, tile;  // tile: launch-wide (counters, partials)
  split_decode(unit, p.n_tiles, p.splits, tile, split);
  const int ltile = w8a8_select_member(p, tile);  // tile within its GEMM (weights, outputs)

  int M = p.M;
  if (p.plan != nullptr) M = min(max(p.plan[0], 0), p.m_grid);
  M = uniform(M);
  const int m0 = mc * BM;
  if (m0 >= M) return;

  const int lane = lane_id(), w = uniform(wave_id()), g = lane >> 4, r = lane & 15;
  const int cw = w % CW, kw = w / CW;
  const int n0 = ltile * BN + cw * BNW;  // first channel of this wave
  const int kb = split * p.k_range;
  const int ke = min(p.K, kb + p.k_range);
  const int nsteps = (ke - kb + 63) / 64;
  // This wave's steps: positions kw, kw + KW, ... of the workgroup's rotated step order.
  const int cnt = nsteps > kw ? (nsteps - kw + KW - 1) / KW : 0;
  const int rot = LAYOUT == 0 ? (int)(((unsigned)tile * 13u + (unsigned)split * 7u) % (unsigned)nsteps) : 0;

  const int m_rows = min(BM, M - m0);
  const rsrc_t asrc = make_rsrc(p.A + (int64_t)m0 * p.lda, (uint32_t)((m_rows - 1) * p.lda + p.K));
  uint32_t arow[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) arow[j] = (j * 16 + r < m_rows) ? (uint32_t)((j * 16 + r) * p.lda + g * 16) : kOOB;

  using WFrag = W8A8WFrag<LAYOUT>;
  constexpr uint32_t FB = W8A8WFragBytes<LAYOUT>::value;  // bytes of one packed fragment
  const int n_rows_w = uniform(max(0, min(BNW, p.N - n0)));
  rsrc_t wsrc;
  uint32_t wrow[RW];
  if constexpr (LAYOUT == 0) {
    wsrc = make_rsrc(p.W + (int64_t)min(n0, p.N - 1) * p.ldw,
                     n_rows_w > 0 ? (uint32_t)((n_rows_w - 1) * p.ldw + p.K) : 0u);
#pragma unroll
    for (int i = 0; i < RW; ++i) wrow[i] = (i * 16 + r < n_rows_w) ? (uint32_t)((i * 16 + r) * p.ldw + g * 16) : kOOB;
  } else {
    // K-step-major packed fragments: (tile t, step s) at fragment s * ntiles + t (FB bytes each).
    const int ntiles = (p.N + 15) / 16;
    const int ksteps = (p.K + 63) / 64;
    wsrc = make_rsrc(p.W, (uint32_t)((size_t)ksteps * ntiles * FB));
#pragma unroll
    for (int i = 0; i < RW; ++i)
      wrow[i] = (n0 / 16 + i < ntiles) ? (uint32_t)((n0 / 16 + i) * FB + lane * (FB / 64)) : kOOB;
  }
  const uint32_t sstride = LAYOUT == 0 ? 64u : (uint32_t)((p.N + 15) / 16) * FB;

  // Per-lane copies of the loop bounds (see w8a8_stream2: wave-uniform bounds turn the load
  // masks into branches, and a branch around a load forces a full vmcnt wait at the join).
  int cnt_v = cnt, ke_v = ke;
  asm volatile("" : "+v"(cnt_v), "+v"(ke_v));

  auto issue = [&](int i, WFrag (&wslot)[RW], v4i (&aslot)[MT]) {
    int pos = kw + i * KW + rot;
    pos = pos >= nsteps ? pos - nsteps : pos;
    const int k0 = kb + pos * 64;
    const bool live = (i < cnt_v) & (k0 + g * 16 < ke_v);
#pragma unroll
    for (int t = 0; t < RW; ++t) {
      const uint32_t off = oob_unless(live & (wrow[t] != kOOB), wrow[t] + (uint32_t)(k0 / 64) * sstride);
      wslot[t] = w8a8_wload<LAYOUT>(wsrc, off);
    }
#pragma unroll
    for (int j = 0; j < MT; ++j)
      aslot[j] = __builtin_amdgcn_raw_buffer_load_b128(asrc, oob_unless(live & (arow[j] != kOOB), arow[j] + (uint32_t)k0), 0, 0);
  };

  const bool owner = kw == 0;
  W8A8EpiScales<MT, RW> es;
  es.load(p, M, m0, n0, owner & (p.splits == 1));

  v4i acc[RW][MT];
#pragma unroll
  for (int t = 0; t < RW; ++t)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[t][j] = v4i{0, 0, 0, 0};

  WFrag wring[NS][RW];
  v4i aring[NS][MT];
  // Prologue: steps 0 .. D-1 in flight, issued in step order.  The scheduling barriers keep
  // the load order identical to the main loop's, so the wait counts the compiler derives at
  // the loop header agree on both incoming paths (otherwise it falls back to vmcnt(0)).
  static_for<0, D>([&](auto sc) {
    constexpr int s = decltype(sc)::value;
    issue(s, wring[s], aring[s]);
    __builtin_amdgcn_sched_barrier(0);
  });
  // Whole turns of the ring; steps past `cnt` load zeros (out-of-range offsets) and their
  // MFMAs add nothing, which keeps the loop body free of branches.
  const int turns = (cnt + NS - 1) / NS;
  for (int it = 0; it < turns; ++it) {
    static_for<0, NS>([&](auto tc) __attribute__((always_inline)) {
      constexpr int t = decltype(tc)::value;
      constexpr int tn = (t + D) % NS;
      issue(it * NS + t + D, wring[tn], aring[tn]);
      __builtin_amdgcn_sched_barrier(0);
      wait_vmcnt<D * PER>();
      if constexpr (t == 0) {
        if (it == 0) tl_mark(p.tl, p.tl_cap, 1);  // diagnostics build: first step landed
      }
#pragma unroll
      for (int a = 0; a < RW; ++a) {
        const v4i wf = w8a8_wop(wring[t][a]);
#pragma unroll
        for (int j = 0; j < MT; ++j)
          acc[a][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf, aring[t][j], acc[a][j], 0, 0, 0);
      }
    });
  }
  wait_vmcnt<0>();
  tl_mark(p.tl, p.tl_cap, 2);  // diagnostics build: main loop done
  if constexpr (LAYOUT == 2) w8a8_unscale16(acc);

  // Reduce the KW waves of each channel group through LDS in one round: each non-owner wave
  // writes its slice, then the owner adds them.
  if constexpr (KW > 1) {
    constexpr int SLICE = BM * BN;  // int32 per slice
    if (kw > 0) {
#pragma unroll
      for (int a = 0; a < RW; ++a)
#pragma unroll
        for (int j = 0; j < MT; ++j)
          *reinterpret_cast<v4i*>(smem_rk + (kw - 1) * SLICE + ((j * 16 + r) * BN + cw * BNW + a * 16 + 4 * g)) = acc[a][j];
    }
    __syncthreads();
    if (owner) {
#pragma unroll
      for (int q = 0; q < KW - 1; ++q)
#pragma unroll
        for (int a = 0; a < RW; ++a)
#pragma unroll
          for (int j = 0; j < MT; ++j)
            acc[a][j] += *reinterpret_cast<const v4i*>(smem_rk + q * SLICE + ((j * 16 + r) * BN + cw * BNW + a * 16 + 4 * g));
    }
  }

  const int cidx = mc * p.n_tiles + tile;
  if (p.splits == 1) {
    if (owner) {
#pragma unroll
      for (int a = 0; a < RW; ++a)
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          const int m = m0 + j * 16 + r, n = n0 + a * 16 + 4 * g;
          if (m < M && n < p.N) w8a8_store4s(p, m, n, acc[a][j], es.a[j], es.w[a]);
        }
    }
    tl_mark(p.tl, p.tl_cap, 3);          // diagnostics build: stores issued
    tl_mark_drained(p.tl, p.tl_cap, 4);  // ... and completed
    return;
  }
  const rsrc_t prs = w8a8_partials_rsrc<BM, BN>(p, cidx);
  if (owner) {
#pragma unroll
    for (int a = 0; a < RW; ++a)
#pragma unroll
      for (int j = 0; j < MT; ++j)
        w8a8_publish_quad<BM, BN>(prs, split, j * 16 + r, cw * BNW + a * 16 + 4 * g, acc[a][j]);
  }
  tl_mark(p.tl, p.tl_cap, 3);  // diagnostics build: partials issued
  __shared__ int s_last_rk;
  w8a8_splitk_finish<BM, BN, NW * 64>(p, prs, cidx, m0, ltile * BN, M, &s_last_rk);
  tl_mark_drained(p.tl, p.tl_cap, 4);  // diagnostics build: hand-off (and, if last, the sum) done
}

template <int MT, int RW, int KW, int NW, int LAYOUT>
__global__ __launch_bounds__(NW * 64) void w8a8_rk_kernel(W8A8Params p) {
  w8a8_rk_body<MT, RW, KW, NW, LAYOUT>(p);
}

}  // namespace specq
