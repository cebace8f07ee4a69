// W4A16 GEMM for gfx950:  C[m, n] = fp16( sum_k a[m,k] * fp16(fp16(q[n,k] - 8) * sc[n, k/G]) )
//
// Follows the arithmetic of the reference Triton kernel (kernels.py:94-135): the unsigned
// nibble minus 8 is converted to fp16 and multiplied by the fp16 group scale in fp16 (one RNE
// rounding), and the dequantized fp16 weights meet the fp16 activations in fp16 x fp16 ->
// fp32 products.  The MI355X schedule:
//
//  * Dequantize once per weight element.  A workgroup's waves each own RW*16 output channels
//    and stream their packed rows straight from HBM into VGPRs (16 bytes = 32 nibbles per lane
//    per 128-wide K block); every nibble is expanded once (v_perm exponent injection, packed
//    fp16 subtract and scale) and the resulting fp16 fragment feeds the MFMAs of all MT token
//    blocks of the workgroup's M-chunk (v_mfma_f32_16x16x32_f16, weights as the A-operand).
//  * The fp16 activations of the M-chunk are DMA'd per K block into an LDS ring and shared
//    by all waves, so they cross L2 once per workgroup rather than once per wave; the packed
//    weights and scales run several K blocks ahead in a register ring (see w4a16_kernel).
//  * Both packed layouts are consumed natively, no repack: layout 0 (reference, kernels.py:89-92)
//    puts k = j and k = j + K/2 in the low/high nibble of byte j; layout 1 packs 8 nibbles per
//    int32 in k order.  The K slots a lane's nibbles stand for are mirrored by the LDS slots
//    its activation fragments are read from, so the MFMA sums the right products.
//  * Split-K across workgroups for small N: fp32 partial tiles are summed by the last
//    workgroup to arrive in split-index order, and the split count depends only on (N, K) and
//    the tile width, never on M or the plan, so eager and plan-mode results are bit-identical.
#pragma once
#include "common.hpp"

namespace specq {

struct W4A16Params {
  const _Float16* A; int64_t lda;
  const uint8_t* Wq; int64_t ldq;     // packed row stride in bytes
  const _Float16* sc; int64_t ld_sc;
  _Float16* C; int64_t ldc;
  const int32_t* plan;
  int M, N, K, group, m_grid;
  int group_shift;        // log2(group)
  int n_tiles, m_chunks, splits;
  int nblocks;            // K / 128
  int blocks_per_split;
  float* partials;        // [m_chunks][n_tiles][splits][BM][BN_wg]
  int32_t* counters;      // [m_chunks][n_tiles]
  int vec_store;
};

// Two unsigned nibbles (bytes of y selected by sel) -> half2 of (nibble + 1024).
__device__ __forceinline__ v2h nib_pair(uint32_t y, uint32_t sel) {
  return __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, y, sel));
}

// Dequantize the 8 weights of MFMA step u from the lane's 16 packed bytes.
template <int LAYOUT>
__device__ __forceinline__ v8h w4_dequant(const v4i& wq, int u, v2h s2) {
  uint32_t y0, y1;
  if constexpr (LAYOUT == 1) {
    const uint32_t x = (uint32_t)wq[u];
    const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
    y0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // nibbles 0..3
    y1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // nibbles 4..7
  } else {
    const uint32_t x0 = (uint32_t)wq[(u & 1) * 2], x1 = (uint32_t)wq[(u & 1) * 2 + 1];
    const int sh = (u >> 1) * 4;
    y0 = (x0 >> sh) & 0x0F0F0F0Fu;
    y1 = (x1 >> sh) & 0x0F0F0F0Fu;
  }
  const v2h bias = {(_Float16)1032.0f, (_Float16)1032.0f};
  v2h h0 = (nib_pair(y0, 0x04010400u) - bias) * s2;
  v2h h1 = (nib_pair(y0, 0x04030402u) - bias) * s2;
  v2h h2 = (nib_pair(y1, 0x04010400u) - bias) * s2;
  v2h h3 = (nib_pair(y1, 0x04030402u) - bias) * s2;
  v8h r;
  r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
  r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
  return r;
}

template <int MT, int RW, int LAYOUT>
struct W4A16Cfg {
  static constexpr int BM = MT * 16, BNW = RW * 16, BN = 4 * BNW;
  static constexpr int NS = LAYOUT == 1 ? 1 : 2;         // scale loads per channel fragment
  static constexpr int LOADS = RW * (1 + NS) + MT;       // vector loads per wave per K block
  static constexpr int A_SLOT = MT * 4 * 1024;            // activation fragments of one K block
  // Blocks in flight: the 63 loads vmcnt counts, 144 KiB of LDS, and 8 ring slots (the number
  // of distinct LDS DMA targets the compiler tracks separately).
  static constexpr int D_CNT = 63 / LOADS - 1;
  static constexpr int D_LDS = (144 * 1024) / A_SLOT - 1;
  static constexpr int D1 = D_CNT < D_LDS ? D_CNT : D_LDS;
  static constexpr int D = D1 > 7 ? 7 : D1;
  static constexpr int NSLOT = D + 1;
  static constexpr int LDS_BYTES = NSLOT * A_SLOT;
  static constexpr bool OK = D >= 1;
  template <int I>
  static constexpr int slot_bytes = I < NSLOT ? A_SLOT : 16;
};

// Global K index of the 8 activations / weights of MFMA step u, lane group g, K block b.
template <int LAYOUT>
__device__ __forceinline__ int w4_k(int b, int u, int g, int halfK) {
  if constexpr (LAYOUT == 1) return 128 * b + 32 * g + 8 * u;
  else return (u < 2 ? 0 : halfK) + 64 * b + 16 * g + 8 * (u & 1);
}

// Pipeline (same scheme as the W8A8 LDS-shared-activation kernel): the 4 waves own RW x 16
// output channels each and walk the split's K blocks together.  Per 128-wide K block a lane
// loads 16 packed bytes (32 nibbles) of its channel row and the group scale(s) into a register
// ring D blocks ahead, while the block's fp16 activation fragments (MT token blocks x 4 MFMA
// steps, 1 KB each, laid out exactly as the B operand reads them) are DMA'd into LDS ring
// slot (b mod (D+1)), one variable per slot, with fence-free barriers.
template <int MT, int RW, int LAYOUT>
__global__ __launch_bounds__(256) void w4a16_kernel(W4A16Params p) {
  using C = W4A16Cfg<MT, RW, LAYOUT>;
  static_assert(C::OK, "need at least one block in flight");
  constexpr int BM = C::BM, BNW = C::BNW, BN = C::BN, D = C::D, NSLOT = C::NSLOT, NS = C::NS;
  __shared__ __attribute__((aligned(16))) uint8_t al0[C::template slot_bytes<0>], al1[C::template slot_bytes<1>],
      al2[C::template slot_bytes<2>], al3[C::template slot_bytes<3>], al4[C::template slot_bytes<4>],
      al5[C::template slot_bytes<5>], al6[C::template slot_bytes<6>], al7[C::template slot_bytes<7>];
  auto slot = [&](auto ic) -> uint8_t* {
    constexpr int i = decltype(ic)::value;
    if constexpr (i == 0) return al0;
    else if constexpr (i == 1) return al1;
    else if constexpr (i == 2) return al2;
    else if constexpr (i == 3) return al3;
    else if constexpr (i == 4) return al4;
    else if constexpr (i == 5) return al5;
    else if constexpr (i == 6) return al6;
    else return al7;
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

  const int lane = lane_id(), w = uniform(wave_id()), g = lane >> 4, r = lane & 15;
  const int n0 = tile * BN + w * BNW;  // first channel of this wave
  const int blk0 = split * p.blocks_per_split;
  const int nblk = max(0, min(p.nblocks, blk0 + p.blocks_per_split) - blk0);
  const int halfK = p.K / 2;
  const int gshift = p.group_shift;

  // Weight and scale slabs of this wave (rows past N read as zero).
  const int rows_w = uniform(max(0, min(BNW, p.N - n0)));
  const int nb = min(n0, p.N - 1);
  const rsrc_t wsrc = make_rsrc(p.Wq + (int64_t)nb * p.ldq, (uint32_t)(rows_w * p.ldq));
  // Scales are fetched as the 4-byte aligned dword holding them: the slab base is rounded
  // down to a dword (sadj halves) and its range up to whole dwords.
  const int64_t sfirst = (int64_t)nb * p.ld_sc;
  const int sadj = (int)(sfirst & 1);
  const rsrc_t ssrc = make_rsrc(p.sc + (sfirst - sadj), (uint32_t)(((rows_w * p.ld_sc + sadj) * 2 + 3) & ~3));
  const int m_rows = min(BM, M - m0);
  const rsrc_t asrc = make_rsrc(p.A + (int64_t)m0 * p.lda, (uint32_t)(((m_rows - 1) * p.lda + p.K) * 2));
  uint32_t arow[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) arow[j] = (16 * j + r < m_rows) ? (uint32_t)((16 * j + r) * p.lda * 2) : kOOB;

  // Per-lane bounds the compiler must treat as non-uniform, so load masks stay selects rather
  // than branches around the loads (a load under a branch costs a full vmcnt(0) at the join).
  int nblk_v = nblk;
  asm volatile("" : "+v"(nblk_v));

  auto w_load = [&](int bl, v4i (&wv)[RW], uint32_t (&sv)[RW][NS]) {
    const int b = blk0 + bl;
    const bool live = bl < nblk_v;
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      const int row = 16 * i + r;
      const bool ok = live & (row < rows_w);
      wv[i] = __builtin_amdgcn_raw_buffer_load_b128(wsrc, oob_unless(ok, (uint32_t)(row * p.ldq + 64 * b + 16 * g)), 0, 0);
#pragma unroll
      for (int h = 0; h < NS; ++h) {
        // The aligned dword holding the fp16 scale (a 16-bit load would be merged into a
        // register the compiler then copies, which waits on the load); the half is picked
        // when the block is consumed.
        const int grp = w4_k<LAYOUT>(b, 2 * h, g, halfK) >> gshift;
        sv[i][h] = __builtin_amdgcn_raw_buffer_load_b32(ssrc, oob_unless(ok, (uint32_t)((row * p.ld_sc + grp + sadj) * 2) & ~3u), 0, 0);
      }
    }
  };
  auto a_issue = [&](int bl, uint8_t* sl) {
    const int k = w4_k<LAYOUT>(blk0 + bl, w, g, halfK);
    const bool live = bl < nblk_v;
#pragma unroll
    for (int j = 0; j < MT; ++j)
      dma16(asrc, sl + (4 * j + w) * 1024, oob_unless(live, arow[j] + (uint32_t)(2 * k)));
  };

  v4f acc[RW][MT];
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  v4i wring[NSLOT][RW];
  uint32_t sring[NSLOT][RW][NS];
  static_for<0, D>([&](auto sc) {
    constexpr int s = decltype(sc)::value;
    w_load(s, wring[s], sring[s]);
    a_issue(s, slot(sc));
    __builtin_amdgcn_sched_barrier(0);  // keep block order: the compiler's wait counts assume it
  });

  for (int b0 = 0; b0 < nblk; b0 += NSLOT) {
    static_for<0, NSLOT>([&](auto tc) __attribute__((always_inline)) {
      constexpr int t = decltype(tc)::value;
      constexpr int tn = (t + D) % NSLOT;
      const int bl = b0 + t;
      w_load(bl + D, wring[tn], sring[tn]);
      a_issue(bl + D, slot(std::integral_constant<int, tn>{}));
      wait_vmcnt<D * C::LOADS>();  // this wave's loads of block bl have landed
      wg_barrier();                // ... and every other wave's activation DMA
      if (bl < nblk) {
        const uint8_t* aslot = slot(tc);
        uint32_t sh16[RW][NS];  // which half of the loaded dword is the scale
#pragma unroll
        for (int i = 0; i < RW; ++i)
#pragma unroll
          for (int h = 0; h < NS; ++h)
            sh16[i][h] = (((16 * i + r) * p.ld_sc + (w4_k<LAYOUT>(blk0 + bl, 2 * h, g, halfK) >> gshift) + sadj) & 1) * 16;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          v8h wf[RW];
#pragma unroll
          for (int i = 0; i < RW; ++i) {
            const _Float16 s = __builtin_bit_cast(_Float16, (uint16_t)(sring[t][i][NS == 1 ? 0 : (u >> 1)] >> sh16[i][NS == 1 ? 0 : (u >> 1)]));
            wf[i] = w4_dequant<LAYOUT>(wring[t][i], u, v2h{s, s});
          }
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            const v8h af = *reinterpret_cast<const v8h*>(aslot + (4 * j + u) * 1024 + lane * 16);
#pragma unroll
            for (int i = 0; i < RW; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[i], af, acc[i][j], 0, 0, 0);
          }
        }
      }
      wg_barrier_lds();  // every wave's reads of slot t are done before it is refilled
    });
  }
  wait_vmcnt<0>();

  typedef _Float16 v4h __attribute__((ext_vector_type(4)));
  auto store4 = [&](int m, int n, v4f v) {
    _Float16* dst = p.C + (int64_t)m * p.ldc + n;
    if (p.vec_store && n + 3 < p.N) {
      v4h o = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
      *reinterpret_cast<v4h*>(dst) = o;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (n + i < p.N) dst[i] = (_Float16)v[i];
    }
  };

  if (p.splits == 1) {
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const int m = m0 + j * 16 + r, n = n0 + i * 16 + 4 * g;
        if (m < M && n < p.N) store4(m, n, acc[i][j]);
      }
    return;
  }

  // Split-K: publish this split's fp32 tile; the last workgroup sums splits in index order.
  const int cidx = mc * p.n_tiles + tile;
  float* base = p.partials + (int64_t)cidx * p.splits * (BM * BN);
  {
    float* mine = base + (int64_t)split * (BM * BN);
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) publish(mine + (j * 16 + r) * BN + w * BNW + i * 16 + 4 * g + c, acc[i][j][c]);
  }
  __shared__ int s_last;
  if (!arrive_last(p.counters + cidx, p.splits, &s_last)) return;
  const int quads = BM * BN / 4;
  for (int q = threadIdx.x; q < quads; q += blockDim.x) {
    const int ml = q / (BN / 4), nl = (q % (BN / 4)) * 4;
    const int m = m0 + ml, n = tile * BN + nl;
    if (m >= M || n >= p.N) continue;
    v4f s = {0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < p.splits; ++sp) {
      const float* src = base + (int64_t)sp * (BM * BN) + ml * BN + nl;
      const v4f t = {collect(src), collect(src + 1), collect(src + 2), collect(src + 3)};
      if (sp == 0) s = t; else s += t;
    }
    store4(m, n, s);
  }
}

}  // namespace specq
