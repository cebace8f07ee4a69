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
//  * The fp16 activations of the M-chunk are staged per K block in LDS (double buffered) and
//    shared by all waves, so they cross L2 once per workgroup rather than once per wave.
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
  int n_tiles, m_chunks, splits;
  int nblocks;            // K / 128
  int blocks_per_split;
  float* partials;        // [m_chunks][n_tiles][splits][BM][BN_wg]
  int32_t* counters;      // [m_chunks][n_tiles]
  int vec_store;
};

constexpr int kW4RowBytes = 256 + 16;  // LDS bytes per staged activation row (128 halves + pad)

// LDS half-slot where MFMA step u of lane group g reads its 8 activations.
template <int LAYOUT>
__device__ __forceinline__ int w4_slot(int u, int g) {
  if constexpr (LAYOUT == 1) return 32 * g + 8 * u;
  else return (u < 2) ? (16 * g + 8 * u) : (64 + 16 * g + 8 * (u - 2));
}

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
__global__ __launch_bounds__(256) void w4a16_kernel(W4A16Params p) {
  constexpr int BM = MT * 16, BNW = RW * 16;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem4[];
  constexpr int nw = 4;
  constexpr int BN = nw * BNW;

  int id = blockIdx.x;
  const int mc = id % p.m_chunks; id /= p.m_chunks;
  const int split = id % p.splits;
  const int tile = id / p.splits;

  int M = p.M;
  if (p.plan != nullptr) M = min(max(p.plan[0], 0), p.m_grid);
  M = uniform(M);
  const int m0 = mc * BM;
  if (m0 >= M) return;

  const int lane = lane_id(), w = wave_id(), g = lane >> 4, r = lane & 15;
  const int n0 = tile * BN + w * BNW;
  const int blk0 = split * p.blocks_per_split;
  const int nblk = max(0, min(p.nblocks, blk0 + p.blocks_per_split) - blk0);
  const int halfK = p.K / 2;

  // Per-lane weight rows and scale rows (rows past N are clamped; their results are dropped).
  const uint8_t* wrow[RW];
  const _Float16* srow[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const int n = min(n0 + i * 16 + r, p.N - 1);
    wrow[i] = p.Wq + (int64_t)n * p.ldq + 16 * g;
    srow[i] = p.sc + (int64_t)n * p.ld_sc;
  }
  // Group index of the lane's K slots in block b.
  auto gidx = [&](int b, int hi) -> int {
    if constexpr (LAYOUT == 1) return (128 * b + 32 * g) / p.group;
    else return (hi ? halfK : 0) + 64 * b + 16 * g;  // divided below
  };

  v4f acc[RW][MT];
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // Activation staging: piece e = tid + t*256 covers row e/16, 16-byte column e%16.
  // The kernel always runs with 4 waves (256 threads), one piece set per wave-row.
  constexpr int threads = 256;
  constexpr int PIECES = BM * 16;
  auto a_src = [&](int b, int e) -> const _Float16* {
    const int row = e >> 4, c = e & 15;
    const int m = min(m0 + row, M - 1);
    int k;
    if constexpr (LAYOUT == 1) k = 128 * b + 8 * c;
    else k = (c < 8) ? (64 * b + 8 * c) : (halfK + 64 * b + 8 * (c - 8));
    return p.A + (int64_t)m * p.lda + k;
  };
  constexpr int MAXP = PIECES / threads;    // = MT
  v4i stage[MAXP];
  auto stage_load = [&](int b) {
#pragma unroll
    for (int t = 0; t < MAXP; ++t) {
      const int e = threadIdx.x + t * threads;
      stage[t] = *reinterpret_cast<const v4i*>(a_src(b, e));
    }
  };
  auto stage_store = [&](int buf) {
    uint8_t* base = smem4 + buf * (BM * kW4RowBytes);
#pragma unroll
    for (int t = 0; t < MAXP; ++t) {
      const int e = threadIdx.x + t * threads;
      *reinterpret_cast<v4i*>(base + (e >> 4) * kW4RowBytes + (e & 15) * 16) = stage[t];
    }
  };

  v4i wcur[RW], wnext[RW];
  v2h scur[RW][2], snext[RW][2];
  auto w_load = [&](int b, v4i (&wv)[RW], v2h (&sv)[RW][2]) {
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      wv[i] = *reinterpret_cast<const v4i*>(wrow[i] + 64 * (int64_t)b);
      if constexpr (LAYOUT == 1) {
        const _Float16 s = srow[i][gidx(b, 0)];
        sv[i][0] = v2h{s, s}; sv[i][1] = sv[i][0];
      } else {
        const _Float16 slo = srow[i][gidx(b, 0) / p.group], shi = srow[i][gidx(b, 1) / p.group];
        sv[i][0] = v2h{slo, slo}; sv[i][1] = v2h{shi, shi};
      }
    }
  };

  if (nblk > 0) {
    stage_load(blk0);
    w_load(blk0, wcur, scur);
    stage_store(0);
    __syncthreads();
  }
  for (int bi = 0; bi < nblk; ++bi) {
    const int b = blk0 + bi;
    const bool more = bi + 1 < nblk;
    if (more) {
      stage_load(b + 1);
      w_load(b + 1, wnext, snext);
    }
    const uint8_t* abase = smem4 + (bi & 1) * (BM * kW4RowBytes);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      v8h wf[RW];
#pragma unroll
      for (int i = 0; i < RW; ++i) wf[i] = w4_dequant<LAYOUT>(wcur[i], u, scur[i][u >> 1]);
      const int slot = w4_slot<LAYOUT>(u, g);
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const v8h af = *reinterpret_cast<const v8h*>(abase + (j * 16 + r) * kW4RowBytes + slot * 2);
#pragma unroll
        for (int i = 0; i < RW; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[i], af, acc[i][j], 0, 0, 0);
      }
    }
    if (more) {
      stage_store((bi + 1) & 1);
#pragma unroll
      for (int i = 0; i < RW; ++i) {
        wcur[i] = wnext[i];
        scur[i][0] = snext[i][0];
        scur[i][1] = snext[i][1];
      }
    }
    __syncthreads();
  }

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
