// W4A16 GEMM, weight-streaming schedule with LDS-shared activations (token tiles of 16 rows
// and more).
//
// Arithmetic and fp32 summation order: w4a16.hpp (reference kernels.py:94-135).
//
//  * Fp16 activations are 4x the bytes per K of the INT4 weight, so for deep token tiles the
//    activation traffic, not the weight stream, is what a schedule must contain.  A workgroup
//    has 8 waves: waves w and w + 4 own the same RW 16-channel fragments of the workgroup's
//    BN = 64 * RW channels, and wave group h = w / 4 sums the blocks of stream h of the split
//    (the 128-wide K blocks at even local index for h = 0, odd for h = 1).  Two waves per
//    SIMD: one wave's dependency and memory stalls hide behind the other's dequant and MFMAs,
//    with the same workgroup count and the same bytes per CU as four waves over all blocks.
//  * Each stream stages its token rows once per chunk of S of its blocks in its own LDS ring
//    of NSLOT slots, filled NSLOT-1 chunks ahead by LDS DMA (buffer_load ... lds), 4 rows x
//    256 bytes per instruction; every activation byte crosses L2 -> CU once per workgroup and
//    is read from LDS by the stream's 4 waves.  Both streams step through their chunks
//    together, one workgroup barrier per chunk.
//  * The DMA lanes fetch 16-byte pieces in an XOR-swizzled order (piece c of row r lands in
//    slot c ^ (r % 16)), so the MFMA-layout ds_read_b128s that consume them are free of bank
//    conflicts.  A K step's MT fragment reads are issued together.
//  * Weights and scales stream from HBM into a register ring NSW blocks deep (a multiple of
//    the S * NSLOT blocks the LDS ring holds); each 16-byte weight load is dequantized once
//    into the A operands of 4 MFMA K steps, each of which meets the MT activation fragments of
//    that step.  Loads past the end are out-of-range buffer reads (zero), so every loop body
//    issues the same loads and all wait counts are compile-time constants.
//  * At the end stream 1's partial tiles go through LDS to stream 0's waves, which add them
//    (even + odd) and store, or hand the sum to split-K.
#pragma once
#include "w4a16.hpp"

namespace specq {

template <int MT, int RW, int S, int NSLOT, int NSW, int LAYOUT>
struct W4WsCfg {
  static constexpr int NSC = W4Nsc<LAYOUT>::value;
  static constexpr int BM = MT * 16, BNW = RW * 16, BN = 4 * BNW;
  static constexpr int SLOT = BM * 256 * S;        // LDS bytes per chunk (256 B of fp16 per row per block)
  static constexpr int P = NSLOT - 1;              // chunks of activation DMA in flight
  static constexpr int A_L = MT * S;               // 1 KB DMA instructions per wave per chunk
  static constexpr int NS = NSW;                   // weight ring slots (blocks) = blocks per loop body
  static constexpr int D = NS - 1;                 // blocks of weights in flight
  static constexpr int WPER = RW * (1 + NSC);      // weight + scale loads per block
  // Loads issued after block i's weights when block i (j = i mod S within its chunk) is
  // consumed: the D later blocks' weights and the DMAs of the chunk starts in (i - D, i].
  static constexpr int wait_w(int j) { return D * WPER + ((D - j + S - 1) / S) * A_L; }
  // Two streams, each with its NSLOT slots; stream 1's tiles are handed over in the two
  // streams' first slots.
  static constexpr bool OK = S >= 1 && NSLOT >= 2 && NSLOT <= 4 && NS % (S * NSLOT) == 0 && NS <= 16 &&
                             wait_w(0) <= 63 && P * S * WPER + P * A_L <= 63 && 2 * NSLOT * SLOT <= 160 * 1024 &&
                             4 * RW * MT * 1024 <= 2 * SLOT;
};

// The kernel body.  `slot_ptr(std::integral_constant<int, i>, h)` returns stream h's
// activation slot i (i < NSLOT, at least SLOT bytes each, 16-byte aligned); the two streams'
// slot 0 must be one contiguous region (slot_ptr(0, 1) == slot_ptr(0, 0) + stride, stride >=
// SLOT), which carries the hand-over at the end.  Separate LDS variables per slot index: the
// compiler's wait-count pass can then tell that reads of one slot do not depend on the DMA
// still filling another.  Also inlined into the plan-mode launch that holds several tilings
// (w4a16_plan.hpp), which passes slots sized for its largest tiling.
template <int MT, int RW, int S, int NSLOT, int NSW, int LAYOUT, class SlotPtr>
__device__ __forceinline__ void w4a16_ws_body(W4A16Params p, SlotPtr slot_ptr) {
  using C = W4WsCfg<MT, RW, S, NSLOT, NSW, LAYOUT>;
  static_assert(C::OK, "unsupported W4A16 weight-stream tile");
  constexpr int BM = C::BM, BNW = C::BNW, BN = C::BN, A_L = C::A_L, NS = C::NS, D = C::D, P = C::P;
  constexpr int WPER = C::WPER, NSC = C::NSC;
  tl_mark(p.tl, p.tl_cap, 0);  // diagnostics build: workgroup start

  int mc, tile, split;
  if (!w4_decode_id(p, mc, tile, split)) return;
  int M = p.M;
  if (p.plan != nullptr) M = min(max(p.plan[0], 0), p.m_grid);
  M = uniform(M);
  const int m0 = mc * BM;
  if (m0 >= M) return;

  const int lane = lane_id(), wv = uniform(wave_id()), g = lane >> 4, r = lane & 15;
  const int h = wv >> 2, w = wv & 3;  // stream, channel group
  const int ltile = w4_select_member(p, tile);  // tile within its GEMM (weights, outputs)
  const int n0 = ltile * BN + w * BNW;
  const int blk0 = split * p.bps;
  const int nblk = max(0, min(p.nblocks, blk0 + p.bps) - blk0);
  // Stream h holds the split's local blocks 2q + h, q = 0 .. nq_h - 1; both streams run
  // stream 0's chunk count (stream 1's last chunk may be past its end).
  const int nq = (nblk - h + 1) >> 1;
  const int nchunks = (((nblk + 1) >> 1) + S - 1) / S;
  int nq_v = nq;
  asm volatile("" : "+v"(nq_v));
  auto blk_of = [&](int q) { return blk0 + 2 * q + h; };

  // ---- Activation DMA.  DMA instruction q (wave w of the stream issues q = w, w + 4, ...)
  // fills block bb = q / (BM/4) of the chunk, rows 4 * (q % (BM/4)) + lane / 16, LDS slot
  // lane % 16 with piece (lane % 16) ^ (row % 16) of the row's 256 bytes of that block.  LDS
  // image: [block][row][16 slots of 16 bytes].  The 16 pieces of block b are the 128
  // activations the block's nibbles stand for: k = 128b + 8c (layouts 1, 2), or k = 64b + 8c
  // (c < 8) and K/2 + 64b + 8(c - 8) (reference layout).
  const int m_rows = min(BM, M - m0);
  const rsrc_t asrc = make_rsrc(p.A + (int64_t)m0 * p.lda, (uint32_t)(((m_rows - 1) * p.lda + p.K) * 2));
  uint32_t dma_off[A_L];  // row byte offset + piece offset within the block (block 0)
  int dma_bb[A_L];
#pragma unroll
  for (int i = 0; i < A_L; ++i) {
    const int q = w + 4 * i;
    const int bb = q / (BM / 4), row = 4 * (q % (BM / 4)) + g;
    const int c = r ^ (row & 15);
    const int piece = LAYOUT == 0 ? (c < 8 ? 16 * c : p.K + 16 * (c - 8)) : 16 * c;
    dma_bb[i] = bb;
    dma_off[i] = row < m_rows ? (uint32_t)(row * p.lda * 2 + piece) : kOOB;
  }
  constexpr int kBlockBytes = LAYOUT == 0 ? 128 : 256;  // activation bytes per block per piece run
  auto dma_chunk = [&](int c, uint8_t* slot) {
#pragma unroll
    for (int i = 0; i < A_L; ++i) {
      const int q = c * S + dma_bb[i];  // the stream's block index
      const bool ok = (q < nq_v) & (dma_off[i] != kOOB);
      dma16(asrc, slot + (w + 4 * i) * 1024, oob_unless(ok, dma_off[i] + (uint32_t)(blk_of(q) * kBlockBytes)));
    }
  };

  W4Weights<RW, LAYOUT> wt;
  wt.init(p, n0);
  auto w_issue = [&](int c, int j, v4i (&wq)[RW], uint32_t (&sv)[RW][NSC]) {
    const int q = c * S + j;
    wt.issue(blk_of(q), q < nq_v, wq, sv);
  };

  v4f acc[RW][MT];
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // Steady state (each stream, its block i = c*S + j): at the top of chunk c the DMA of chunk
  // c + P is issued (into LDS slot (c + P) % NSLOT); each block issues the weights of block
  // i + D into ring slot (i + D) % NS and consumes block i.  In issue order, the DMA of chunk y
  // belongs to block (y - P) * S (ahead of that block's weights) and the weights of block x to
  // block x - D.  The prologue issues everything belonging to the blocks before 0 in that
  // order, so every wait count below is a compile-time constant:
  //   after block i's weights:  D weight blocks + the DMAs of chunk starts in (i - D, i];
  //   after chunk c's DMA:      P*S weight blocks + P-1 DMA groups.
  v4i wring[NS][RW];
  uint32_t sring[NS][RW][NSC];
  constexpr int T0 = (P * S > D ? P * S : D);  // the prologue covers blocks -T0 .. -1
  static_for<0, T0>([&](auto tc) {
    constexpr int t = decltype(tc)::value - T0;  // block time t < 0
    if constexpr (t % S == 0 && t / S + P >= 0) {
      constexpr int y = t / S + P;
      dma_chunk(y, slot_ptr(std::integral_constant<int, y % NSLOT>{}, h));
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (t + D >= 0) {
      constexpr int x = t + D;
      w_issue(x / S, x % S, wring[x % NS], sring[x % NS]);
      __builtin_amdgcn_sched_barrier(0);
    }
  });

  // Piece of MFMA step u for lane group g within a block's 16 pieces.
  int pc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) pc[u] = LAYOUT == 0 ? ((u < 2 ? 0 : 8) + 2 * g + (u & 1)) : 4 * g + u;

  // Loop body: NS blocks = NS / S chunks, so LDS slots and ring slots are compile-time.
  constexpr int CPB = NS / S;  // chunks per body
  for (int c0 = 0; c0 < nchunks; c0 += CPB) {
    static_for<0, CPB>([&](auto cc_) __attribute__((always_inline)) {
      constexpr int cb = decltype(cc_)::value;
      constexpr int cl = cb % NSLOT;
      const int c = c0 + cb;
      wait_vmcnt<P * S * WPER + (P - 1) * A_L>();  // this wave's DMA of chunk c has landed
      wg_barrier_lds();  // ... every wave's has, and nobody reads slot (c + P) % NSLOT any more
      if constexpr (cb == 0) {
        if (c0 == 0) tl_mark(p.tl, p.tl_cap, 1);  // diagnostics build: first chunk landed
      }
      dma_chunk(c + P, slot_ptr(std::integral_constant<int, (cl + P) % NSLOT>{}, h));
      __builtin_amdgcn_sched_barrier(0);
      const uint8_t* aslot = slot_ptr(std::integral_constant<int, cl>{}, h);
      static_for<0, S>([&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        constexpr int ri = (cb * S + j) % NS;
        constexpr int rn = (cb * S + j + D) % NS;
        constexpr int jn = (j + D) % S;
        constexpr int cn = (j + D) / S;
        w_issue(c + cn, jn, wring[rn], sring[rn]);
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<C::wait_w(j)>();
        const int b = blk_of(c * S + j);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          // The step's MT activation fragments are read first, so their LDS latency overlaps
          // (with each other and with the dequantization of the weight fragments) instead of
          // standing between every pair of MFMAs.
          v8h af[MT];
#pragma unroll
          for (int t = 0; t < MT; ++t)
            af[t] = *reinterpret_cast<const v8h*>(aslot + (j * BM + 16 * t + r) * 256 + 16 * (pc[u] ^ r));
          __builtin_amdgcn_sched_barrier(0);
          v8h wf[RW];
#pragma unroll
          for (int i = 0; i < RW; ++i) wf[i] = wt.frag(b, i, u, wring[ri], sring[ri]);
#pragma unroll
          for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int i = 0; i < RW; ++i) acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[i], af[t], acc[i][t], 0, 0, 0);
        }
      });
    });
  }
  wait_vmcnt<0>();
  tl_mark(p.tl, p.tl_cap, 2);  // diagnostics build: main loop done

  // Hand-over: stream 1's tiles into the streams' first slots (every wave is past its last
  // read of the rings), stream 0 adds them: even + odd.
  __syncthreads();
  float* xch = reinterpret_cast<float*>(slot_ptr(std::integral_constant<int, 0>{}, 0)) + w * (RW * MT * 256);
  if (h == 1) {
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j) *reinterpret_cast<v4f*>(xch + ((i * MT + j) * 64 + lane) * 4) = acc[i][j];
  }
  __syncthreads();
  if (h == 0) {
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j) acc[i][j] = acc[i][j] + *reinterpret_cast<const v4f*>(xch + ((i * MT + j) * 64 + lane) * 4);
  }

  // The split-K arrival flag lives in stream 0's slot 1, free once the main loop is done (the
  // hand-over above uses the streams' slot 0), so the workgroup's LDS is exactly its rings:
  // two 80-row workgroups (4 x 20 KB each) then fit one CU.
  int* s_last_ws4 = reinterpret_cast<int*>(slot_ptr(std::integral_constant<int, 1>{}, 0));
  if (p.splits == 1) {
    if (h == 0) {
#pragma unroll
      for (int i = 0; i < RW; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          const int m = m0 + 16 * j + r, n = n0 + 16 * i + 4 * g;
          if (m < M && n < p.N) w4_store4(p, m, n, acc[i][j]);
        }
    }
    tl_mark(p.tl, p.tl_cap, 3);          // diagnostics build: stores issued
    tl_mark_drained(p.tl, p.tl_cap, 4);  // ... and completed
    return;
  }
  const int cidx = mc * p.n_tiles + tile;
  const rsrc_t prs = w4_partials_rsrc<BM, BN>(p, cidx);
  if (h == 0) {
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j) w4_publish_quad<BM, BN>(prs, split, 16 * j + r, w * BNW + 16 * i + 4 * g, acc[i][j]);
  }
  tl_mark(p.tl, p.tl_cap, 3);  // diagnostics build: partials issued
  // Every thread of the workgroup takes part in the arrival and the last one's finish.
  w4_splitk_finish<BM, BN, 512>(p, prs, cidx, m0, ltile * BN, M, s_last_ws4);
  tl_mark_drained(p.tl, p.tl_cap, 4);  // diagnostics build: hand-off (and, if last, the sum) done
}

constexpr int kW4WsThreads = 512;  // the split-K finish above is instantiated for 512 threads

template <int MT, int RW, int S, int NSLOT, int NSW, int LAYOUT>
__global__ __launch_bounds__(kW4WsThreads) void w4a16_ws_kernel(W4A16Params p) {
  constexpr int SLOT = W4WsCfg<MT, RW, S, NSLOT, NSW, LAYOUT>::SLOT;
  __shared__ __attribute__((aligned(16))) uint8_t lds_s0[2][SLOT], lds_s1[2][SLOT];
  __shared__ __attribute__((aligned(16))) uint8_t lds_s2[2][NSLOT > 2 ? SLOT : 16], lds_s3[2][NSLOT > 3 ? SLOT : 16];
  w4a16_ws_body<MT, RW, S, NSLOT, NSW, LAYOUT>(p, [&](auto ic, int h) -> uint8_t* {
    constexpr int i = decltype(ic)::value;
    if constexpr (i == 0) return lds_s0[h];
    else if constexpr (i == 1) return lds_s1[h];
    else if constexpr (i == 2) return lds_s2[h];
    else return lds_s3[h];
  });
}

}  // namespace specq
