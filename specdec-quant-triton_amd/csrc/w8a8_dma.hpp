// W8A8 GEMM, LDS-DMA streaming schedule for 16-byte aligned operands (the fast path).
//
// Same arithmetic as w8a8_kernel (reference kernels.py:27-55: INT32 accumulation, then
// (acc * sa[m]) * sw[n] in fp32, one RNE cast to fp16), different schedule:
//
//  * The weights and the activation tile are streamed HBM -> LDS with gfx950's direct
//    buffer_load_dwordx4 ... lds, in K chunks of KC bytes through a ring of NSTAGE slots.
//    No VGPRs are spent on data in flight, so a CU keeps 48-64 KB of weights moving while
//    it computes, the depth a full-bandwidth HBM stream needs.
//  * DRAM-friendly fetch, MFMA-friendly read: each DMA instruction covers 4 rows x 256
//    contiguous bytes (measured ~1.6x faster than the 16 rows x 64 bytes an MFMA operand
//    spans), and an XOR swizzle of 16-byte chunks lets the MFMA side read its 16 rows x 64
//    bytes per K step from LDS without bank conflicts.
//  * Workgroup = 4 waves arranged NWN x NWK: NWN waves own different output channels
//    (RW x 16 each) and share the activation fragments; NWK waves split the chunk's K steps
//    and are reduced through LDS at the end.
//  * Range checking of the buffer descriptors zero-fills rows past N / past the active M
//    and K past the split, so every wave issues the same number of DMA loads per chunk and
//    one compile-time s_waitcnt vmcnt covers them.
//  * Split-K across workgroups and plan mode work as in w8a8_kernel (device-coherent partial
//    tiles, last workgroup to arrive applies the epilogue).
#pragma once
#include "w8a8.hpp"

namespace specq {

template <int MT, int RW, int NWN>
struct W8A8DmaCfg {
  static constexpr int NWK = 4 / NWN;
  static constexpr int FR = NWN * RW + MT;                 // 16-row fragments (weights + tokens)
  static constexpr int STEPS = FR <= 3 ? 8 : 4;            // 64-byte K steps per chunk (x4 = blocks)
  static constexpr int KC = STEPS * 64;
  static constexpr int FB = FR * STEPS;                    // KiB per ring slot
  static constexpr int WSTEPS = STEPS / NWK;               // steps a wave computes per chunk
  static constexpr int LOADS = FB / 4;                     // DMA instructions per wave per chunk
  // Ring depth: small tiles aim for two workgroups per CU (80 KiB each), large ones for one;
  // all slots but one are in flight, bounded by the 63 loads vmcnt can count.
  static constexpr int LDS_CAP_KB = FR <= 6 ? 80 : 152;   // 152: leaves room for static LDS
  static constexpr int NS_LDS = LDS_CAP_KB / FB;
  static constexpr int NS_CNT = 63 / LOADS;
  static constexpr int NS_MIN = NS_LDS < NS_CNT ? NS_LDS : NS_CNT;
  static constexpr int NSTAGE = NS_MIN > 8 ? 8 : NS_MIN;
  static constexpr int BM = MT * 16, BNW = RW * 16, BN = NWN * BNW;
  static constexpr int LDW = BNW + kW8A8Pad;               // reduction slice pitch (int32)
  static constexpr int DATA_BYTES = NSTAGE * FB * 1024;
  static constexpr int RED_BYTES = NWK > 1 ? NWN * BM * LDW * 4 : 0;
  static constexpr int LDS_BYTES = DATA_BYTES > RED_BYTES ? DATA_BYTES : RED_BYTES;
  static_assert(NSTAGE >= 2, "need at least double buffering");
  static_assert(NSTAGE * LOADS <= 63, "vmcnt holds at most 63 outstanding loads");
  static_assert(STEPS % 4 == 0 && WSTEPS >= 1 && WSTEPS * NWK == STEPS, "chunk = whole 256-byte blocks");
};

// LDS layout of one 16-row fragment in a chunk: STEPS/4 blocks of 16 rows x 256 bytes,
// row-major, with the 16-byte column chunk c of row r stored at chunk slot c ^ r.  The DMA
// side fills a block with 4 instructions of 4 rows x 256 contiguous bytes each (long DRAM
// runs); the MFMA side reads, for K step s, chunk 4*(s%4) + lane/16 of row lane%16, which
// the XOR spreads over all 16 chunk slots (no bank conflicts).
__device__ __forceinline__ uint32_t frag_read_off(int s, int lane) {
  const int r = lane & 15, c = 4 * (s & 3) + (lane >> 4);
  return (uint32_t)((s >> 2) * 4096 + r * 256 + ((c ^ r) & 15) * 16);
}


template <int MT, int RW, int NWN>
__global__ __launch_bounds__(256) void w8a8_dma_kernel(W8A8Params p) {
  using C = W8A8DmaCfg<MT, RW, NWN>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];

  int id = blockIdx.x;
  const int mc = id % p.m_chunks; id /= p.m_chunks;
  const int split = id % p.splits;
  const int tile = id / p.splits;

  int M = p.M;
  if (p.plan != nullptr) M = min(max(p.plan[0], 0), p.m_grid);
  M = uniform(M);
  const int m0 = mc * C::BM;
  if (m0 >= M) return;

  const int lane = lane_id(), w = wave_id(), g = lane >> 4, r = lane & 15;
  const int wn = w % NWN, wk = w / NWN;
  const int n0 = tile * C::BN;
  const int kb = split * p.k_range;
  const int ke = min(p.K, kb + p.k_range);
  const int nchunks = (ke - kb + C::KC - 1) / C::KC;

  const int n_rows = min(C::BN, p.N - n0), m_rows = min(C::BM, M - m0);
  const rsrc_t wsrc = make_rsrc(p.W + (int64_t)n0 * p.ldw, (uint32_t)((n_rows - 1) * p.ldw + p.K));
  const rsrc_t asrc = make_rsrc(p.A + (int64_t)m0 * p.lda, (uint32_t)((m_rows - 1) * p.lda + p.K));

  // DMA assignment: wave w fetches rows 4w..4w+3 of every 16-row block of every fragment;
  // lane l takes row 4w + l/16 and the column chunk (l%16) ^ row, i.e. the bytes the reader
  // expects in LDS slot l of the instruction.  Fragment f < NWN*RW is weight channel block f,
  // the rest are token blocks of the activations.
  const int drow = 4 * w + (lane >> 4);                 // row within a 16-row fragment
  const uint32_t dcol = (uint32_t)(((lane & 15) ^ drow) * 16);
  uint32_t frow[C::FR];
#pragma unroll
  for (int f = 0; f < C::FR; ++f) {
    if (f < NWN * RW) {
      const int row = f * 16 + drow;
      frow[f] = row < n_rows ? (uint32_t)(row * p.ldw) + dcol : kOOB;
    } else {
      const int row = (f - NWN * RW) * 16 + drow;
      frow[f] = row < m_rows ? (uint32_t)(row * p.lda) + dcol : kOOB;
    }
  }

  auto issue = [&](int c, int slot) {
    const int kc = kb + c * C::KC;
    uint8_t* sbase = lds8 + (size_t)slot * (C::FB * 1024) + w * 1024;
#pragma unroll
    for (int f = 0; f < C::FR; ++f) {
      const rsrc_t rs = f < NWN * RW ? wsrc : asrc;
#pragma unroll
      for (int blk = 0; blk < C::STEPS / 4; ++blk) {
        const int k = kc + blk * 256;                     // + column chunk, checked below
        const uint32_t off = (frow[f] != kOOB && k + (int)dcol < ke) ? frow[f] + k : kOOB;
        dma16(rs, sbase + (f * C::STEPS + blk * 4) * 1024, off);
      }
    }
  };

  v4i acc[RW][MT];
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  // Ring of NSTAGE chunk slots: chunks c+1 .. c+NSTAGE-1 are in flight while chunk c is
  // computed.  Prefetches past the end are out of range and only write zeros to free slots.
#pragma unroll
  for (int c = 0; c < C::NSTAGE - 1; ++c) issue(c, c);
  for (int c = 0; c < nchunks; ++c) {
    const int cn = c + C::NSTAGE - 1;
    issue(cn, cn % C::NSTAGE);    // the slot chunk c-1 used; freed by the last barrier
    wait_vmcnt<(C::NSTAGE - 1) * C::LOADS>();  // this wave's loads of chunk c have landed
    __syncthreads();              // ... and every other wave's
    const uint8_t* buf = lds8 + (size_t)(c % C::NSTAGE) * C::FB * 1024;
#pragma unroll
    for (int t = 0; t < C::WSTEPS; ++t) {
      const int s = wk + t * C::NWK;
      const uint32_t ro = frag_read_off(s, lane);
      v4i wf[RW], af[MT];
#pragma unroll
      for (int i = 0; i < RW; ++i)
        wf[i] = *reinterpret_cast<const v4i*>(buf + (size_t)((wn * RW + i) * C::STEPS) * 1024 + ro);
#pragma unroll
      for (int j = 0; j < MT; ++j)
        af[j] = *reinterpret_cast<const v4i*>(buf + (size_t)((NWN * RW + j) * C::STEPS) * 1024 + ro);
      w8a8_mma_step<MT, RW>(wf, af, acc);
    }
    __syncthreads();              // slot c % NSTAGE is refilled by the next iteration
  }
  wait_vmcnt<0>();                // drain the final (all out-of-range) prefetch before reusing LDS
  __syncthreads();

  // Reduce the NWK waves sharing a channel block (wave wk = 0 keeps the sum).
  if constexpr (C::NWK > 1) {
    int32_t* slice = reinterpret_cast<int32_t*>(lds8) + wn * (C::BM * C::LDW);
    for (int src = C::NWK - 1; src >= 1; --src) {
      if (wk == src) {
#pragma unroll
        for (int i = 0; i < RW; ++i)
#pragma unroll
          for (int j = 0; j < MT; ++j)
            *reinterpret_cast<v4i*>(slice + (j * 16 + r) * C::LDW + i * 16 + 4 * g) = acc[i][j];
      }
      __syncthreads();
      if (wk == 0) {
#pragma unroll
        for (int i = 0; i < RW; ++i)
#pragma unroll
          for (int j = 0; j < MT; ++j)
            acc[i][j] += *reinterpret_cast<const v4i*>(slice + (j * 16 + r) * C::LDW + i * 16 + 4 * g);
      }
      __syncthreads();
    }
  }

  const int cidx = mc * p.n_tiles + tile;
  const int nw0 = n0 + wn * C::BNW;  // first channel of this wave's block
  if (p.splits == 1) {
    if (wk == 0) {
#pragma unroll
      for (int i = 0; i < RW; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          const int m = m0 + j * 16 + r, n = nw0 + i * 16 + 4 * g;
          if (m < M && n < p.N) w8a8_store4(p, m, n, acc[i][j]);
        }
    }
    return;
  }

  int32_t* base = p.partials + (int64_t)cidx * p.splits * (C::BM * C::BN);
  if (wk == 0) {
    int32_t* mine = base + (int64_t)split * (C::BM * C::BN);
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          publish(mine + (j * 16 + r) * C::BN + wn * C::BNW + i * 16 + 4 * g + c, acc[i][j][c]);
  }
  __shared__ int s_last;
  if (!arrive_last(p.counters + cidx, p.splits, &s_last)) return;
  constexpr int QUADS = C::BM * C::BN / 4;
  for (int q = threadIdx.x; q < QUADS; q += blockDim.x) {
    const int ml = q / (C::BN / 4), nl = (q % (C::BN / 4)) * 4;
    const int m = m0 + ml, n = n0 + nl;
    if (m >= M || n >= p.N) continue;
    v4i s = {0, 0, 0, 0};
    for (int sp = 0; sp < p.splits; ++sp) {
      const int32_t* src = base + (int64_t)sp * (C::BM * C::BN) + ml * C::BN + nl;
      s += v4i{collect(src), collect(src + 1), collect(src + 2), collect(src + 3)};
    }
    w8a8_store4(p, m, n, s);
  }
}

}  // namespace specq
