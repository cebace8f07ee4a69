// W8A8 GEMM, register-streaming schedule with DRAM-friendly weight fetches (aligned fast path).
//
// Same arithmetic as w8a8_kernel (reference kernels.py:27-55: INT32 accumulation, then
// (acc * sa[m]) * sw[n] in fp32, one RNE cast to fp16).  The schedule is built around how
// MI355X HBM wants to be read:
//
//  * A load instruction whose 64 lanes cover 16 rows x 64 bytes (the MFMA operand shape)
//    streams a [N, K] weight at ~60% of the rate of one covering 4 rows x 256 contiguous bytes
//    (measured on 56 MB).  So the weight is fetched in 256-byte K blocks of 16 rows, four
//    instructions of 4 rows x 256 B each, into VGPRs (double-buffered batches of UB blocks),
//    and each wave transposes its own blocks to MFMA layout through a private LDS tile: one
//    ds_write_b128 and four ds_read_b128 per lane per block, XOR-swizzled (16-byte chunk c of
//    row r at slot c ^ r) so both directions are bank-conflict free.  No barriers: a wave
//    only reads what it wrote.
//  * LAYOUT 1 takes the weight pre-packed into MFMA fragments ([N/16][K/64][64 lanes x 16 B],
//    packed by specq_w8a8_pack_weight): every instruction then reads 1 KB contiguous straight into
//    operand registers and the LDS transpose is skipped.
//  * Waves of a workgroup split the workgroup's K range into contiguous block ranges and are
//    reduced through LDS; split-K across workgroups, plan mode and the epilogue are shared
//    with w8a8_kernel.
#pragma once
#include "w8a8.hpp"

namespace specq {

template <int MT, int RW>
struct W8A8StreamCfg {
  // Blocks (4 K steps) per register batch: about 128 VGPRs for both buffers together.
  static constexpr int PER_BLOCK = 4 * (RW + MT);          // v4i registers per block
  static constexpr int raw = 16 / PER_BLOCK;
  static constexpr int UB = raw < 1 ? 1 : (raw > 4 ? 4 : raw);
  static constexpr int BM = MT * 16, BN = RW * 16;
  static constexpr int LDW = BN + kW8A8Pad;
};

// Offset of chunk c of row r inside a 16 x 256-byte XOR-swizzled block.
__device__ __forceinline__ uint32_t swz(int r, int c) { return (uint32_t)(r * 256 + ((c ^ r) & 15) * 16); }

template <int MT, int RW, int LAYOUT>
__global__ __launch_bounds__(256) void w8a8_stream_kernel(W8A8Params p) {
  using C = W8A8StreamCfg<MT, RW>;
  constexpr int BM = C::BM, BN = C::BN, UB = C::UB, LDW = C::LDW;
  extern __shared__ __attribute__((aligned(16))) int32_t smem_s[];

  const int nw = blockDim.x / kWave;
  int id = blockIdx.x;
  const int mc = id % p.m_chunks; id /= p.m_chunks;
  const int split = id % p.splits;
  const int tile = id / p.splits;

  int M = p.M;
  if (p.plan != nullptr) M = min(max(p.plan[0], 0), p.m_grid);
  M = uniform(M);
  const int m0 = mc * BM;
  if (m0 >= M) return;

  const int n0 = tile * BN;
  const int kb = split * p.k_range;
  const int ke = min(p.K, kb + p.k_range);
  const int lane = lane_id(), w = wave_id(), g = lane >> 4, r = lane & 15;

  // This wave's contiguous range of 256-byte K blocks inside [kb, ke).
  const int nblk_wg = (ke - kb + 255) / 256;
  const int per_wave = (nblk_wg + nw - 1) / nw;
  const int blk_begin = min(w * per_wave, nblk_wg);
  const int blk_end = min(blk_begin + per_wave, nblk_wg);
  const int nbatch = (blk_end - blk_begin + UB - 1) / UB;

  const int n_rows = min(BN, p.N - n0), m_rows = min(BM, M - m0);
  // Weight descriptor: row-major slab of this tile, or its packed fragment run.
  rsrc_t wsrc;
  uint32_t woff[RW];
  if constexpr (LAYOUT == 0) {
    wsrc = make_rsrc(p.W + (int64_t)n0 * p.ldw, (uint32_t)((n_rows - 1) * p.ldw + p.K));
    // Fetch lane (row 4q + g, column chunk r) of block instruction q.
#pragma unroll
    for (int i = 0; i < RW; ++i) woff[i] = (uint32_t)(i * 16 * p.ldw);
  } else {
    // Packed: fragment (row tile t, K step s) is 1 KB at (t * ksteps + s) * 1024.
    const int ksteps = (p.K + 63) / 64;
    const int64_t t0 = n0 / 16;
    const int ntiles = (p.N + 15) / 16;
    const int tiles_here = min(RW, ntiles - (int)t0);
    wsrc = make_rsrc(p.W + t0 * ksteps * 1024, (uint32_t)(tiles_here * ksteps * 1024));
#pragma unroll
    for (int i = 0; i < RW; ++i) woff[i] = i < tiles_here ? (uint32_t)(i * ksteps * 1024) : kOOB;
  }
  const rsrc_t asrc = make_rsrc(p.A + (int64_t)m0 * p.lda, (uint32_t)((m_rows - 1) * p.lda + p.K));
  uint32_t aoff[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) aoff[j] = (j * 16 + r < m_rows) ? (uint32_t)((j * 16 + r) * p.lda) : kOOB;

  // Row-major fetch geometry: instruction q of a block covers rows 4q .. 4q+3.
  const int frow = 4 * 0 + g;  // row within the quad (add 4q)
  uint8_t* stage = reinterpret_cast<uint8_t*>(smem_s) + (size_t)w * RW * 4096;

  v4i acc[RW][MT];
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  v4i wa[UB][RW][4], aa[UB][4][MT], wb[UB][RW][4], ab[UB][4][MT];
  auto load_batch = [&](int bt, v4i (&wv)[UB][RW][4], v4i (&av)[UB][4][MT]) {
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int blk = blk_begin + bt * UB + u;
      const bool live = blk < blk_end;
      const int kblk = kb + blk * 256;
#pragma unroll
      for (int i = 0; i < RW; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint32_t off = kOOB;
          if constexpr (LAYOUT == 0) {
            const int row = i * 16 + 4 * q + frow;
            const int k = kblk + r * 16;
            if (live && row < n_rows && k < ke) off = (uint32_t)((4 * q + frow) * p.ldw + k) + woff[i];
          } else {
            const int s = kblk / 64 + q;  // K step
            if (live && woff[i] != kOOB && kblk + q * 64 < ke) off = woff[i] + (uint32_t)(s * 1024 + lane * 16);
          }
          wv[u][i][q] = __builtin_amdgcn_raw_buffer_load_b128(wsrc, off, 0, 0);
        }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int k = kblk + q * 64 + g * 16;
#pragma unroll
        for (int j = 0; j < MT; ++j)
          av[u][q][j] = __builtin_amdgcn_raw_buffer_load_b128(asrc, (live && k < ke) ? aoff[j] + k : kOOB, 0, 0);
      }
    }
  };
  auto mma_batch = [&](v4i (&wv)[UB][RW][4], v4i (&av)[UB][4][MT]) {
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      v4i wf[RW][4];
      if constexpr (LAYOUT == 0) {
        // Transpose the block through this wave's LDS tile: lane (row 4q+g, chunk r) writes
        // its 16 bytes; lane (row r, chunk 4s+g) reads the K step s operand.
#pragma unroll
        for (int i = 0; i < RW; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<v4i*>(stage + i * 4096 + swz(4 * q + g, r)) = wv[u][i][q];
#pragma unroll
        for (int i = 0; i < RW; ++i)
#pragma unroll
          for (int s = 0; s < 4; ++s)
            wf[i][s] = *reinterpret_cast<const v4i*>(stage + i * 4096 + swz(r, 4 * s + g));
      } else {
#pragma unroll
        for (int i = 0; i < RW; ++i)
#pragma unroll
          for (int s = 0; s < 4; ++s) wf[i][s] = wv[u][i][s];
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < RW; ++i)
#pragma unroll
          for (int j = 0; j < MT; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[i][s], av[u][s][j], acc[i][j], 0, 0, 0);
    }
  };

  load_batch(0, wa, aa);
  for (int bt = 0; bt < nbatch; bt += 2) {
    load_batch(bt + 1, wb, ab);
    mma_batch(wa, aa);
    load_batch(bt + 2, wa, aa);
    mma_batch(wb, ab);
  }

  // Cross-wave reduction (one LDS slice, waves nw-1 .. 1 deposit in turn, wave 0 sums).
  __syncthreads();  // every wave is past its last use of the transpose tiles
  for (int src = nw - 1; src >= 1; --src) {
    if (w == src) {
#pragma unroll
      for (int i = 0; i < RW; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j)
          *reinterpret_cast<v4i*>(smem_s + (j * 16 + r) * LDW + i * 16 + 4 * g) = acc[i][j];
    }
    __syncthreads();
    if (w == 0) {
#pragma unroll
      for (int i = 0; i < RW; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j)
          acc[i][j] += *reinterpret_cast<const v4i*>(smem_s + (j * 16 + r) * LDW + i * 16 + 4 * g);
    }
    __syncthreads();
  }

  const int cidx = mc * p.n_tiles + tile;
  if (p.splits == 1) {
    if (w == 0) {
#pragma unroll
      for (int i = 0; i < RW; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          const int m = m0 + j * 16 + r, n = n0 + i * 16 + 4 * g;
          if (m < M && n < p.N) w8a8_store4(p, m, n, acc[i][j]);
        }
    }
    return;
  }
  int32_t* base = p.partials + (int64_t)cidx * p.splits * (BM * BN);
  if (w == 0) {
    int32_t* mine = base + (int64_t)split * (BM * BN);
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) publish(mine + (j * 16 + r) * BN + i * 16 + 4 * g + c, acc[i][j][c]);
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
