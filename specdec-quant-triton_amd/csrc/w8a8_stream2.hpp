// W8A8 GEMM, register-streaming weights + LDS-shared activations (aligned path, deeper M tiles).
//
// Same arithmetic as w8a8_kernel (reference kernels.py:27-55).  Schedule for BLOCK_M >= 32,
// where the activation fragments dominate a per-wave register budget:
//
//  * The 4 waves of a workgroup own different output channels (RW x 16 each) and walk the
//    same K range, so they share the activation tile.  Each 256-byte K block of the tile
//    (MT x 4 MFMA fragments, L2 resident) is DMA'd into LDS (buffer_load ... lds), one
//    fragment per instruction, lane l fetching the 16 bytes it will read back.  That keeps
//    activations out of VGPRs entirely.
//  * The freed registers hold a ring of D weight blocks per wave (RW x 4 KB each) fetched
//    4 rows x 256 contiguous bytes per instruction (or 1 KB packed fragments, LAYOUT 1), so a
//    CU keeps on the order of 100 KB of weights in flight.  Row-major blocks are transposed
//    to MFMA layout through a private XOR-swizzled LDS tile per wave, as in w8a8_stream.
//  * Weights and activations of a block are issued together, D blocks ahead, into register
//    ring slot and LDS ring slot (b mod (D+1)).  Every iteration issues the same loads
//    (range-checked to zero past the end), so one compile-time s_waitcnt vmcnt separates the
//    block being computed from the D blocks in flight.
//  * Each LDS ring slot is its own __shared__ variable and the main loop is unrolled over the
//    slots at compile time: the compiler can then tell the slots apart and waits only for
//    the DMA into the slot it reads, instead of for all of them.  Barriers are s_barrier
//    without a memory fence (wg_barrier), because __syncthreads() would drain every
//    outstanding load at each block.
#pragma once
#include "w8a8_dma.hpp"
#include "w8a8_stream.hpp"

namespace specq {

template <int MT, int RW, int LAYOUT>
struct W8A8Stream2Cfg {
  static constexpr int BM = MT * 16, BNW = RW * 16, BN = 4 * BNW;
  static constexpr int LOADS = 4 * RW + MT;              // vector loads per wave per block
  static constexpr int A_SLOT = MT * 4 * 1024;            // activation bytes per block
  static constexpr int T_BYTES = LAYOUT == 0 ? 4 * RW * 4096 : 0;  // per-wave transpose tiles
  // Blocks in flight: weights (registers) and activations (LDS) run the same D blocks ahead,
  // bounded by the 63 loads vmcnt can count, ~128 VGPRs of weight blocks and 152 KiB of LDS.
  static constexpr int D_CNT = 63 / LOADS - 1;
  static constexpr int D_REG = 8 / RW - 1;
  static constexpr int D_LDS = (152 * 1024 - T_BYTES) / A_SLOT - 1;
  static constexpr int D1 = D_CNT < D_REG ? D_CNT : D_REG;
  static constexpr int D2 = D1 < D_LDS ? D1 : D_LDS;
  static constexpr int D = D2 > 6 ? 6 : D2;
  static constexpr int NSLOT = D + 1;
  static constexpr int LDS_BYTES = NSLOT * A_SLOT + T_BYTES;
  static constexpr bool OK = D >= 1;  // tiles with no room for a block in flight are not built
  template <int I>
  static constexpr int slot_bytes = I < NSLOT ? A_SLOT : 16;
};

template <int MT, int RW, int LAYOUT>
__global__ __launch_bounds__(256) void w8a8_stream2_kernel(W8A8Params p) {
  using C = W8A8Stream2Cfg<MT, RW, LAYOUT>;
  static_assert(C::OK, "need at least one block in flight");
  constexpr int BM = C::BM, BNW = C::BNW, BN = C::BN, D = C::D, NSLOT = C::NSLOT;
  // LDS ring: one variable per slot (see above); unused ones are never referenced.
  __shared__ __attribute__((aligned(16))) uint8_t sl0[C::template slot_bytes<0>], sl1[C::template slot_bytes<1>],
      sl2[C::template slot_bytes<2>], sl3[C::template slot_bytes<3>], sl4[C::template slot_bytes<4>],
      sl5[C::template slot_bytes<5>], sl6[C::template slot_bytes<6>];
  __shared__ __attribute__((aligned(16))) uint8_t tstage_all[C::T_BYTES > 0 ? C::T_BYTES : 16];
  auto slot = [&](auto ic) -> uint8_t* {
    constexpr int i = decltype(ic)::value;
    if constexpr (i == 0) return sl0;
    else if constexpr (i == 1) return sl1;
    else if constexpr (i == 2) return sl2;
    else if constexpr (i == 3) return sl3;
    else if constexpr (i == 4) return sl4;
    else if constexpr (i == 5) return sl5;
    else return sl6;
  };

  int id = blockIdx.x;
  const int mc = id % p.m_chunks; id /= p.m_chunks;
  const int split = id % p.splits;
  const int tile = id / p.splits;

  int M = p.M;
  if (p.plan != nullptr) M = min(max(p.plan[0], 0), p.m_grid);
  M = uniform(M);
  const int m0 = mc * BM;
  if (m0 >= M) return;

  // The wave index is made an SGPR value: descriptors and LDS DMA bases derived from it must be
  // wave-uniform, or the compiler emits a per-lane waterfall loop around every load.
  const int lane = lane_id(), w = uniform(wave_id()), g = lane >> 4, r = lane & 15;
  const int n0 = tile * BN;
  const int nw0 = n0 + w * BNW;  // first channel of this wave
  const int kb = split * p.k_range;
  const int ke = min(p.K, kb + p.k_range);
  const int nblk = (ke - kb + 255) / 256;

  const int m_rows = min(BM, M - m0);
  const rsrc_t asrc = make_rsrc(p.A + (int64_t)m0 * p.lda, (uint32_t)((m_rows - 1) * p.lda + p.K));
  // Activation fragment (token block u, K step w) of a block: row 16u + r, bytes 16g.. of the step.
  uint32_t arow[MT];
#pragma unroll
  for (int u = 0; u < MT; ++u) {
    const int row = u * 16 + r;
    arow[u] = row < m_rows ? (uint32_t)(row * p.lda + g * 16) : kOOB;
  }

  // Weight slab of this wave.  Clamps are folded into v_med3 (a VALU op) by the compiler;
  // readfirstlane keeps the descriptor in SGPRs.
  const int n_rows_w = uniform(max(0, min(BNW, p.N - nw0)));
  rsrc_t wsrc;
  uint32_t woff[RW];
  if constexpr (LAYOUT == 0) {
    wsrc = make_rsrc(p.W + (int64_t)min(nw0, p.N - 1) * p.ldw,
                     n_rows_w > 0 ? (uint32_t)((n_rows_w - 1) * p.ldw + p.K) : 0u);
#pragma unroll
    for (int i = 0; i < RW; ++i) woff[i] = (uint32_t)(i * 16 * p.ldw);
  } else {
    const int ksteps = (p.K + 63) / 64;
    const int ntiles = (p.N + 15) / 16;
    const int t0 = min(nw0 / 16, ntiles - 1);
    const int tiles_here = uniform(max(0, min(RW, ntiles - nw0 / 16)));
    wsrc = make_rsrc(p.W + (int64_t)t0 * ksteps * 1024, (uint32_t)(tiles_here * ksteps * 1024));
#pragma unroll
    for (int i = 0; i < RW; ++i) woff[i] = i < tiles_here ? (uint32_t)(i * ksteps * 1024) : kOOB;
  }

  uint8_t* tstage = tstage_all + w * RW * 4096;

  // Copies of the block count and K end that the compiler must treat as per-lane values:
  // with wave-uniform bounds it turns the load masks into branches around the loads, and a
  // load under a branch makes it wait for every outstanding load (vmcnt(0)) at the join.  The
  // masks below use '&' rather than '&&' for the same reason.
  int nblk_v = nblk, ke_v = ke;
  asm volatile("" : "+v"(nblk_v), "+v"(ke_v));

  auto w_load = [&](int blk, v4i (&wv)[RW][4]) {
    const int kblk = kb + blk * 256;
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t off = kOOB;
        if constexpr (LAYOUT == 0) {
          const int row = i * 16 + 4 * q + g;
          const int k = kblk + r * 16;
          if ((blk < nblk_v) & (row < n_rows_w) & (k < ke_v)) off = woff[i] + (uint32_t)((4 * q + g) * p.ldw + k);
        } else {
          if ((blk < nblk_v) & (woff[i] != kOOB) & (kblk + q * 64 < ke_v))
            off = woff[i] + (uint32_t)((kblk / 64 + q) * 1024 + lane * 16);
        }
        wv[i][q] = __builtin_amdgcn_raw_buffer_load_b128(wsrc, off, 0, 0);
      }
  };
  auto a_issue = [&](int blk, uint8_t* sl) {
    const int k = kb + blk * 256 + w * 64;
#pragma unroll
    for (int u = 0; u < MT; ++u)
      dma16(asrc, sl + (4 * u + w) * 1024,
            ((blk < nblk_v) & (arow[u] != kOOB) & (k + g * 16 < ke_v)) ? arow[u] + k : kOOB);
  };

  v4i acc[RW][MT];
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  v4i ring[NSLOT][RW][4];
  // Prologue: blocks 0 .. D-1 in flight, issued in block order (the scheduling barriers keep
  // the compiler from hoisting the DMAs above the weight loads, which would leave its own
  // wait counts for the weight registers stricter than the pipeline needs).
  static_for<0, D>([&](auto sc) {
    constexpr int s = decltype(sc)::value;
    w_load(s, ring[s]);
    a_issue(s, slot(sc));
    __builtin_amdgcn_sched_barrier(0);
  });

  // Main loop, unrolled over the NSLOT ring slots.  Iteration b issues block b+D (weights into
  // the register slot and activations into the LDS slot that block b-1 used), waits until only
  // blocks b+1 .. b+D are outstanding, computes block b.
  for (int b0 = 0; b0 < nblk; b0 += NSLOT) {
    static_for<0, NSLOT>([&](auto tc) __attribute__((always_inline)) {
      constexpr int t = decltype(tc)::value;
      constexpr int tn = (t + D) % NSLOT;
      const int b = b0 + t;
      w_load(b + D, ring[tn]);
      a_issue(b + D, slot(std::integral_constant<int, tn>{}));
      wait_vmcnt<D * C::LOADS>();  // this wave's loads of block b have landed
      wg_barrier();                // ... and every other wave's activation DMA
      if (b < nblk) {
        const uint8_t* aslot = slot(tc);
        v4i wf[RW][4];
        if constexpr (LAYOUT == 0) {
#pragma unroll
          for (int i = 0; i < RW; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              *reinterpret_cast<v4i*>(tstage + i * 4096 + swz(4 * q + g, r)) = ring[t][i][q];
#pragma unroll
          for (int i = 0; i < RW; ++i)
#pragma unroll
            for (int s = 0; s < 4; ++s) wf[i][s] = *reinterpret_cast<const v4i*>(tstage + i * 4096 + swz(r, 4 * s + g));
        } else {
#pragma unroll
          for (int i = 0; i < RW; ++i)
#pragma unroll
            for (int s = 0; s < 4; ++s) wf[i][s] = ring[t][i][s];
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          v4i af[MT];
#pragma unroll
          for (int j = 0; j < MT; ++j) af[j] = *reinterpret_cast<const v4i*>(aslot + (4 * j + s) * 1024 + lane * 16);
#pragma unroll
          for (int i = 0; i < RW; ++i)
#pragma unroll
            for (int j = 0; j < MT; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[i][s], af[j], acc[i][j], 0, 0, 0);
        }
      }
      wg_barrier_lds();  // every wave's reads of LDS slot t are done before iteration b+1 refills it
    });
  }
  wait_vmcnt<0>();  // drain out-of-range prefetches

  const int cidx = mc * p.n_tiles + tile;
  if (p.splits == 1) {
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const int m = m0 + j * 16 + r, n = nw0 + i * 16 + 4 * g;
        if (m < M && n < p.N) w8a8_store4(p, m, n, acc[i][j]);
      }
    return;
  }
  int32_t* base = p.partials + (int64_t)cidx * p.splits * (BM * BN);
  {
    int32_t* mine = base + (int64_t)split * (BM * BN);
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) publish(mine + (j * 16 + r) * BN + w * BNW + i * 16 + 4 * g + c, acc[i][j][c]);
  }
  __shared__ int s_last;
  if (!arrive_last(p.counters + cidx, p.splits, &s_last)) return;
  constexpr int QUADS = BM * BN / 4;
  for (int q = threadIdx.x; q < QUADS; q += blockDim.x) {
    const int ml = q / (BN / 4), nl = (q % (BN / 4)) * 4;
    const int m = m0 + ml, n = n0 + nl;
    if (m >= M || n >= p.N) continue;
    v4i s = {0, 0, 0, 0};
    for (int sp = 0; sp < p.splits; ++sp) {
      const int32_t* src = base + (int64_t)sp * (BM * BN) + ml * BN + nl;
      s += v4i{collect(src), collect(src + 1), collect(src + 2), collect(src + 3)};
    }
    w8a8_store4(p, m, n, s);
  }
}

}  // namespace specq
