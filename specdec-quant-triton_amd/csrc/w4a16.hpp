// W4A16 GEMM for gfx950:  C[m, n] = fp16( sum_k a[m,k] * fp16(fp16(q[n,k] - 8) * sc[n, k/G]) )
//
// Arithmetic of the reference Triton kernel (kernels.py:94-135): the unsigned nibble minus 8
// is converted to fp16 and multiplied by the fp16 group scale in fp16 (one RNE rounding), and
// the dequantized fp16 weights meet the fp16 activations in fp16 x fp16 -> fp32 products
// (v_mfma_f32_16x16x32_f16, weights as the A operand) summed into an fp32 accumulator.
//
// Pieces shared by the two kernel families (w4a16_rk.hpp: activations loaded straight into
// MFMA operand registers, for 16-row token tiles; w4a16_ws.hpp: activations staged in an LDS
// ring shared by the waves of a workgroup, for deeper tiles):
//
//  * K is walked in 128-wide blocks.  For every block a lane loads 16 packed bytes (32
//    nibbles) of its weight row and expands them into the A operands of 4 MFMA K steps.  The
//    K indices a lane's nibbles stand for (w4_k) fix which activations the B operand holds.
//    Weight layouts, consumed natively:
//      0  reference uint8 [N, K/2] (kernels.py:89-92): byte j holds k = j and k = j + K/2;
//      1  int32 [N, K/8], 8 nibbles per word in k order;
//      2  packed at load time (w4a16_pack_kernel): 1 KB MFMA fragments, fragment (b, t) of
//         K block b and 16-row tile t at (b * ntiles + t) KB, so a wave's block is one
//         contiguous 1 KB load and the workgroups running together sweep one window.  Within
//         a word the 8 nibbles sit where fp16 magic constants extract them without byte
//         shuffles (w4_dequant).
//  * The fp32 summation order is fixed by (N, K), the split count and the K order of the
//    layout (layouts 1 and 2 share one; layout 0's blocks pair k with k + K/2): split s takes
//    a contiguous range of blocks and sums it as two streams, the blocks at even and at odd
//    local index, each starting from zero in increasing block order (4 MFMA K steps per
//    block, in order); the split's result is even + odd, and the splits are added in split
//    order by the last workgroup to arrive.  Token tiling, channel tiling, kernel family and
//    plan mode never change it, so every tile choice and plan-mode replay produces
//    bit-identical results.
#pragma once
#include "common.hpp"

namespace specq {

constexpr int kW4MaxGroup = 4;  // GEMMs of one grouped launch

struct W4A16Params {
  const _Float16* A; int64_t lda;
  const uint8_t* Wq; int64_t ldq;  // row stride in bytes (layouts 0, 1)
  const _Float16* sc; int64_t ld_sc;
  _Float16* C; int64_t ldc;
  const int32_t* plan;
  int M, N, K, m_grid;
  int group_shift;       // log2(group)
  int n_tiles;           // channel tiles of BN
  int m_chunks, splits;
  int units;             // n_tiles * splits
  int nblocks, bps;      // K / 128 blocks; blocks per split
  int ntiles16;          // 16-row tiles (packed layout)
  float* partials;       // [m_chunks][n_tiles][splits][BM][BN] when splits > 1
  int32_t* counters;     // [m_chunks][n_tiles]
  int vec_store;
  // Grouped launch: n_grp GEMMs sharing A (and K, group, splits), member 0 in the fields
  // above and member g >= 1 in grp_*[g - 1]; member g owns launch-wide channel tiles
  // [grp_tile_end[g - 2] (0 for g = 0), grp_tile_end[g - 1]).
  int n_grp;
  int grp_tile_end[kW4MaxGroup - 1];
  const uint8_t* grp_Wq[kW4MaxGroup - 1];
  int64_t grp_ldq[kW4MaxGroup - 1];
  const _Float16* grp_sc[kW4MaxGroup - 1];
  int64_t grp_ld_sc[kW4MaxGroup - 1];
  _Float16* grp_C[kW4MaxGroup - 1];
  int64_t grp_ldc[kW4MaxGroup - 1];
  int grp_N[kW4MaxGroup - 1], grp_ntiles16[kW4MaxGroup - 1], grp_vec_store[kW4MaxGroup - 1];
  uint64_t* tl;  // diagnostics build only: per-workgroup timestamps (null otherwise)
  int tl_cap;    // workgroups tl has room for
};

// Points the weight, scale and output fields of p at the GEMM of a grouped launch that owns
// launch-wide channel tile `tile`, and returns the tile's index within that GEMM.  The member
// is picked with scalar selects (the parameter block is never indexed dynamically).  Split-K
// counters and partial tiles stay indexed by the launch-wide tile.
__device__ __forceinline__ int w4_select_member(W4A16Params& p, int tile) {
  if (p.n_grp <= 1) return tile;
  int first = 0;
#pragma unroll
  for (int g = 1; g < kW4MaxGroup; ++g) {
    if (g < p.n_grp && tile >= p.grp_tile_end[g - 1]) {  // g is a constant once unrolled
      first = p.grp_tile_end[g - 1];
      p.Wq = p.grp_Wq[g - 1]; p.ldq = p.grp_ldq[g - 1];
      p.sc = p.grp_sc[g - 1]; p.ld_sc = p.grp_ld_sc[g - 1];
      p.C = p.grp_C[g - 1]; p.ldc = p.grp_ldc[g - 1];
      p.N = p.grp_N[g - 1]; p.ntiles16 = p.grp_ntiles16[g - 1]; p.vec_store = p.grp_vec_store[g - 1];
    }
  }
  return tile - first;
}


// Two unsigned nibbles (bytes of y selected by sel) -> half2 of (nibble + 1024).
__device__ __forceinline__ v2h nib_pair(uint32_t y, uint32_t sel) {
  return __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, y, sel));
}

// The 8 dequantized weights of MFMA K step u from a lane's 16 packed bytes.  s2 holds the
// scale twice.  (1024 + n) - 1032 = n - 8 exactly; the product is the one rounding.
//
// Layout 2 word (w4a16_pack_kernel): weights j = 0..7 of the step at nibble positions
// 0, 4, 1, 5, 2, 6, 3, 7 (bits 4p..4p+3), i.e. the pairs (0,1), (2,3), (4,5), (6,7) at bits
// {0-3, 16-19}, {4-7, 20-23}, {8-11, 24-27}, {12-15, 28-31}.  One AND-OR per pair turns a
// pair into two fp16: a nibble in bits 0-3 of a half under exponent 0x64 is 1024 + n (ulp 1),
// a nibble in bits 4-7 under exponent 0x54 is 64 + n (ulp 1/16); the upper two pairs take one
// shift first.  Subtracting 1032 or 72 gives n - 8 exactly, so every layout dequantizes to the
// same fp16 values.
//
// v_and_or_b32 is a VOP3 instruction, which takes no literal on this architecture, so the
// compiler would split (x & m) | c into two VOP2 instructions with literals; the masks go in
// scalar registers and the exponent patterns in (loop-invariant) vector registers instead.
__device__ __forceinline__ uint32_t and_or_b32(uint32_t x, uint32_t mask, uint32_t bits) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(bits));
  return r;
}

__device__ __forceinline__ v8h w4_dequant_packed(uint32_t x, v2h s2) {
  const uint32_t y = x >> 8;
  const v2h b1024 = {(_Float16)1032.0f, (_Float16)1032.0f};
  const v2h b64 = {(_Float16)72.0f, (_Float16)72.0f};
  const v2h h0 = (__builtin_bit_cast(v2h, and_or_b32(x, 0x000F000Fu, 0x64006400u)) - b1024) * s2;
  const v2h h1 = (__builtin_bit_cast(v2h, and_or_b32(x, 0x00F000F0u, 0x54005400u)) - b64) * s2;
  const v2h h2 = (__builtin_bit_cast(v2h, and_or_b32(y, 0x000F000Fu, 0x64006400u)) - b1024) * s2;
  const v2h h3 = (__builtin_bit_cast(v2h, and_or_b32(y, 0x00F000F0u, 0x54005400u)) - b64) * s2;
  v8h r;
  r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
  r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
  return r;
}

template <int LAYOUT>
__device__ __forceinline__ v8h w4_dequant(const v4i& wq, int u, v2h s2) {
  if constexpr (LAYOUT == 2) {
    return w4_dequant_packed((uint32_t)wq[u], s2);
  } else {
    uint32_t y0, y1;  // nibbles of weights 0..3 and 4..7, one per byte
    if constexpr (LAYOUT == 1) {
      const uint32_t x = (uint32_t)wq[u];
      const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
      y0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
      y1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
    } else {
      const uint32_t x0 = (uint32_t)wq[(u & 1) * 2], x1 = (uint32_t)wq[(u & 1) * 2 + 1];
      const int sh = (u >> 1) * 4;
      y0 = (x0 >> sh) & 0x0F0F0F0Fu;
      y1 = (x1 >> sh) & 0x0F0F0F0Fu;
    }
    const v2h bias = {(_Float16)1032.0f, (_Float16)1032.0f};
    const v2h h0 = (nib_pair(y0, 0x04010400u) - bias) * s2;
    const v2h h1 = (nib_pair(y0, 0x04030402u) - bias) * s2;
    const v2h h2 = (nib_pair(y1, 0x04010400u) - bias) * s2;
    const v2h h3 = (nib_pair(y1, 0x04030402u) - bias) * s2;
    v8h r;
    r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
    r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
    return r;
  }
}

// First of the 8 K indices of MFMA step u for lane group g in block b.
template <int LAYOUT>
__device__ __forceinline__ int w4_k(int b, int u, int g, int halfK) {
  if constexpr (LAYOUT == 0) return (u < 2 ? 0 : halfK) + 64 * b + 16 * g + 8 * (u & 1);
  else return 128 * b + 32 * g + 8 * u;
}
// Scale loads per lane per block: layout 0 spans two K ranges (low and high nibbles).
template <int LAYOUT>
struct W4Nsc { static constexpr int value = LAYOUT == 0 ? 2 : 1; };

// Per-wave weight and scale addressing for RW 16-row fragments starting at channel n0.
template <int RW, int LAYOUT>
struct W4Weights {
  static constexpr int NSC = W4Nsc<LAYOUT>::value;
  rsrc_t wsrc, ssrc;
  uint32_t wrow[RW];     // byte offset of the lane's row (or fragment) at block 0, or kOOB
  int32_t srow[RW];      // scale element index of the lane's row (dword-aligned base), -1 if none
  int halfK, gshift, g;
  uint32_t bstride;      // bytes between consecutive blocks of one fragment

  __device__ __forceinline__ void init(const W4A16Params& p, int n0) {
    const int lane = lane_id(), r = lane & 15;
    g = lane >> 4;
    halfK = p.K / 2;
    gshift = p.group_shift;
    const int rows_w = uniform(max(0, min(RW * 16, p.N - n0)));
    const int nb = min(n0, p.N - 1);
    if constexpr (LAYOUT == 2) {
      wsrc = make_rsrc(p.Wq, (uint32_t)((size_t)p.nblocks * p.ntiles16 * 1024));
#pragma unroll
      for (int i = 0; i < RW; ++i)
        wrow[i] = (n0 / 16 + i < p.ntiles16) ? (uint32_t)((n0 / 16 + i) * 1024 + lane * 16) : kOOB;
      bstride = (uint32_t)p.ntiles16 * 1024u;
    } else {
      wsrc = make_rsrc(p.Wq + (int64_t)nb * p.ldq, rows_w > 0 ? (uint32_t)((rows_w - 1) * p.ldq + p.K / 2) : 0u);
#pragma unroll
      for (int i = 0; i < RW; ++i)
        wrow[i] = (16 * i + r < rows_w) ? (uint32_t)((16 * i + r) * p.ldq + 16 * g) : kOOB;
      bstride = 64;
    }
    // Scales are fetched as the 4-byte aligned dword holding them: the slab base is rounded
    // down to a dword (sadj halves) and its range up to whole dwords.
    const int64_t sfirst = (int64_t)nb * p.ld_sc;
    const int sadj = (int)(sfirst & 1);
    ssrc = make_rsrc(p.sc + (sfirst - sadj), rows_w > 0 ? (uint32_t)((((rows_w - 1) * p.ld_sc + (p.K >> gshift) + sadj) * 2 + 3) & ~3) : 0u);
#pragma unroll
    for (int i = 0; i < RW; ++i) srow[i] = (16 * i + r < rows_w) ? (int32_t)((16 * i + r) * p.ld_sc + sadj) : -1;
  }
  // Loads of block b (live: inside this wave's range).  NT loads: the weight is streamed once.
  __device__ __forceinline__ void issue(int b, bool live, v4i (&wv)[RW], uint32_t (&sv)[RW][NSC]) const {
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      const bool ok = live & (wrow[i] != kOOB);
      const bool oks = live & (srow[i] >= 0);
      wv[i] = __builtin_amdgcn_raw_buffer_load_b128(wsrc, oob_unless(ok, wrow[i] + (uint32_t)b * bstride), 0, 2);
#pragma unroll
      for (int h = 0; h < NSC; ++h) {
        const int e = srow[i] + (w4_k<LAYOUT>(b, 2 * h, g, halfK) >> gshift);
        sv[i][h] = __builtin_amdgcn_raw_buffer_load_b32(ssrc, oob_unless(oks, (uint32_t)(e * 2) & ~3u), 0, 0);
      }
    }
  }
  // Dequantized A operand of fragment i, MFMA step u, from block b's loads.
  __device__ __forceinline__ v8h frag(int b, int i, int u, const v4i (&wv)[RW], const uint32_t (&sv)[RW][NSC]) const {
    const int h = NSC == 1 ? 0 : (u >> 1);
    const int e = srow[i] + (w4_k<LAYOUT>(b, 2 * h, g, halfK) >> gshift);
    const _Float16 s = __builtin_bit_cast(_Float16, (uint16_t)(sv[i][h] >> ((e & 1) * 16)));
    return w4_dequant<LAYOUT>(wv[i], u, v2h{s, s});
  }
};

// Output quad: 4 consecutive channels of one token row.
__device__ __forceinline__ void w4_store4(const W4A16Params& p, int m, int n, v4f v) {
  _Float16* dst = p.C + (int64_t)m * p.ldc + n;
  if (p.vec_store && n + 3 < p.N) {
    *reinterpret_cast<v4h*>(dst) = v4h{(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (n + i < p.N) dst[i] = (_Float16)v[i];
  }
}

// Workgroup -> (M-chunk, channel tile, split); false for padding workgroups.
__device__ __forceinline__ bool w4_decode_id(const W4A16Params& p, int& mc, int& tile, int& split) {
  int unit;
  // Eager launches run the M-chunks of a channel tile together on one XCD (W4A16 at M = 288:
  // q|k|v 43.1 -> 39.0 us, gate|up 92.0 -> 89.6; M = 200 gate|up 69.9 -> 66.4); plan mode keeps
  // the chunks in order so those past the active M are the last dispatched and exit at once.
  if (p.plan == nullptr && p.m_chunks > 1) {
    if (!interleaved_unit(p.m_chunks, p.units, mc, unit)) return false;
  } else if (!chunked_unit(p.m_chunks, p.units, mc, unit)) {
    return false;
  }
  split_decode(unit, p.n_tiles, p.splits, tile, split);
  return true;
}

// Split-K hand-off of a workgroup's fp32 tile [BM][BN] (row = token), 16 bytes per lane.
template <int BM, int BN>
__device__ __forceinline__ rsrc_t w4_partials_rsrc(const W4A16Params& p, int cidx) {
  return make_rsrc(p.partials + (int64_t)cidx * p.splits * (BM * BN), (uint32_t)(p.splits * BM * BN * 4));
}
template <int BM, int BN>
__device__ __forceinline__ void w4_publish_quad(rsrc_t prs, int split, int ml, int nl, v4f v) {
  publish16(prs, (uint32_t)(((split * BM + ml) * BN + nl) * 4), __builtin_bit_cast(v4i, v));
}
// The last workgroup of the tile to arrive adds the splits in split order (0, 1, 2, ...).
// Thread t owns quads t, t + NT, ...; the partials of up to QG quads x SB splits are loaded
// together, so the sum costs one memory round trip per group of quads.
template <int BM, int BN, int NT>
__device__ __forceinline__ void w4_splitk_finish(const W4A16Params& p, rsrc_t prs, int cidx, int m0, int nbase,
                                                 int M, int* s_last) {
  if (!arrive_last(p.counters + cidx, p.splits, s_last, p.tl, p.tl_cap)) return;
  constexpr int QUADS = BM * BN / 4;
  constexpr int QPT = (QUADS + NT - 1) / NT;  // quads per thread
  constexpr int QG = QPT <= 4 ? QPT : 4;      // quads summed together
  constexpr int SB = 16 / QG > 8 ? 8 : 16 / QG;  // splits loaded together
#pragma unroll
  for (int g0 = 0; g0 < QPT; g0 += QG) {
    int ml[QG], nl[QG];
    bool ok[QG];
#pragma unroll
    for (int i = 0; i < QG; ++i) {
      const int q = (int)threadIdx.x + (g0 + i) * NT;
      ml[i] = q / (BN / 4);
      nl[i] = (q % (BN / 4)) * 4;
      ok[i] = (g0 + i < QPT) & (q < QUADS) & (m0 + ml[i] < M) & (nbase + nl[i] < p.N);
    }
    v4f s[QG];
    for (int sp0 = 0; sp0 < p.splits; sp0 += SB) {
      v4i t[QG][SB];
#pragma unroll
      for (int i = 0; i < QG; ++i)
#pragma unroll
        for (int u = 0; u < SB; ++u)
          t[i][u] = collect16(prs, oob_unless(ok[i] & (sp0 + u < p.splits),
                                              (uint32_t)((((sp0 + u) * BM + ml[i]) * BN + nl[i]) * 4)));
#pragma unroll
      for (int i = 0; i < QG; ++i)
#pragma unroll
        for (int u = 0; u < SB; ++u) {
          const v4f v = __builtin_bit_cast(v4f, t[i][u]);
          if (sp0 + u == 0) s[i] = v;
          else if (sp0 + u < p.splits) s[i] += v;
        }
    }
#pragma unroll
    for (int i = 0; i < QG; ++i)
      if (ok[i]) w4_store4(p, m0 + ml[i], nbase + nl[i], s[i]);
  }
}

// Epilogue shared by the families: store the wave's fp32 tiles, or hand them to split-K.
// `tile` is the launch-wide channel tile (counters, partials); n0_wave - nl_wave is the first
// channel of the tile within its GEMM.
template <int MT, int RW, int BM, int BN>
__device__ __forceinline__ void w4_epilogue(const W4A16Params& p, const v4f (&acc)[RW][MT], int mc, int tile, int split,
                                            int m0, int n0_wave, int nl_wave, int M, int* s_last) {
  const int lane = lane_id(), g = lane >> 4, r = lane & 15;
  if (p.splits == 1) {
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const int m = m0 + 16 * j + r, n = n0_wave + 16 * i + 4 * g;
        if (m < M && n < p.N) w4_store4(p, m, n, acc[i][j]);
      }
    tl_mark(p.tl, p.tl_cap, 3);          // diagnostics build: stores issued
    tl_mark_drained(p.tl, p.tl_cap, 4);  // ... and completed
    return;
  }
  const int cidx = mc * p.n_tiles + tile;
  const rsrc_t prs = w4_partials_rsrc<BM, BN>(p, cidx);
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) w4_publish_quad<BM, BN>(prs, split, 16 * j + r, nl_wave + 16 * i + 4 * g, acc[i][j]);
  tl_mark(p.tl, p.tl_cap, 3);  // diagnostics build: partials issued
  w4_splitk_finish<BM, BN, 256>(p, prs, cidx, m0, n0_wave - nl_wave, M, s_last);
  tl_mark_drained(p.tl, p.tl_cap, 4);  // diagnostics build: hand-off (and, if last, the sum) done
}

}  // namespace specq
