// W8A8 GEMM for gfx950:  C[m, n] = fp16( (float(sum_k A[m,k] * W[n,k]) * sa[m]) * sw[n] )
//
// Follows the arithmetic of the reference Triton kernel (kernels.py:27-55): INT8 x INT8
// products accumulated exactly in INT32, then the per-token and per-channel scales applied
// left to right in fp32, then one RNE cast to fp16.  The schedule is MI355X-specific:
//
//  * Weight-streaming orientation.  W (the large operand) is the MFMA A-operand and is loaded
//    straight from HBM into VGPRs, 16 contiguous bytes per lane per 64-wide K step, so each
//    weight byte crosses the memory system once per M-chunk.  The activations (small, L2
//    resident) are the MFMA B-operand.  v_mfma_i32_16x16x64_i8 produces a 16(n) x 16(m) tile.
//  * A workgroup owns BN = RW*16 output channels and one M-chunk of BM = MT*16 tokens, which
//    it keeps in INT32 accumulators for its whole K range.  With BLOCK_M >= M the weights are
//    read exactly once; smaller BLOCK_M re-reads them once per M-chunk like the reference.
//  * The waves of a workgroup split its K range (interleaved 64-byte steps, so the waves of
//    one workgroup read adjacent memory), then reduce their accumulators through LDS.
//  * To fill 256 CUs the K range is further split across workgroups (split-K).  INT32 sums are
//    order independent, so the split is exact by construction: each split publishes its INT32
//    partial tile with device-coherent stores, and the last workgroup to arrive (agent-scope
//    atomic counter, no cache-wide fence) sums the partials, applies the epilogue and resets
//    the counter, so the workspace needs no memset between calls and the kernel is legal
//    inside a captured graph.
//  * Plan mode: the active M is read from a device int32 (plan[0]) and clamped to the rows
//    the grid was sized for; M-chunks at or beyond it exit before touching memory, so one
//    graph captured at the maximum grid replays every M and never writes rows >= M.
#pragma once
#include "common.hpp"

namespace specq {

struct W8A8Params {
  const int8_t* A; int64_t lda;
  const int8_t* W; int64_t ldw;
  const float* sa; const float* sw;
  __half* C; int64_t ldc;
  const int32_t* plan;
  int M, N, K;
  int m_grid;          // rows the grid covers (grid_m_max, or M)
  int n_tiles, m_chunks, splits;
  int k_range;         // K bytes per split, a multiple of 64
  int32_t* partials;   // [m_chunks][n_tiles][splits][BM*BN] when splits > 1
  int32_t* counters;   // [m_chunks][n_tiles], zero between calls
  int vec_store;       // 1 when C rows allow 8-byte aligned stores of 4 halves
  // Grouped launch: n_grp GEMMs that share A, sa, M and K (q, k and v; gate and up), each with
  // its own weight, channel scales, output and N.  Member 0 is W / ldw / sw / C / ldc / N above;
  // members 1.. are the grp_* entries.  n_tiles counts the tiles of every member, and tile t
  // belongs to member g when grp_tile_end[g-1] <= t < grp_tile_end[g].
  int n_grp;
  int grp_tile_end[3];
  const int8_t* grp_W[3];
  int64_t grp_ldw[3];
  const float* grp_sw[3];
  __half* grp_C[3];
  int64_t grp_ldc[3];
  int grp_N[3];
  int grp_vec_store[3];
  uint64_t* tl;        // diagnostics build only: per-workgroup timestamps (null otherwise)
  int tl_cap;          // workgroups tl has room for
};
constexpr int kW8A8MaxGroup = 4;

// Points W, ldw, sw, C, ldc and N at the GEMM of a grouped launch that owns launch-wide tile
// `tile`, and returns the tile's index within that GEMM.  The member is picked with scalar
// selects (the parameter block is never indexed dynamically).  Counters and split-K partials
// stay indexed by the launch-wide tile.
__device__ __forceinline__ int w8a8_select_member(W8A8Params& p, int tile) {
  if (p.n_grp <= 1) return tile;
  int first = 0;
#pragma unroll
  for (int g = 1; g < kW8A8MaxGroup; ++g) {
    if (g < p.n_grp && tile >= p.grp_tile_end[g - 1]) {  // g is a constant once unrolled
      first = p.grp_tile_end[g - 1];
      p.W = p.grp_W[g - 1]; p.ldw = p.grp_ldw[g - 1]; p.sw = p.grp_sw[g - 1];
      p.C = p.grp_C[g - 1]; p.ldc = p.grp_ldc[g - 1]; p.N = p.grp_N[g - 1];
      p.vec_store = p.grp_vec_store[g - 1];
    }
  }
  return tile - first;
}

constexpr int kW8A8Pad = 4;  // int32 padding per LDS row

// K steps per register batch: about 160 VGPRs of double-buffered operands, at most 8.
template <int MT, int RW>
struct W8A8Unroll {
  static constexpr int raw = 20 / (MT + RW);
  static constexpr int value = raw < 1 ? 1 : (raw > 8 ? 8 : raw);
};

template <int MT, int RW>
__device__ __forceinline__ void w8a8_mma_step(const v4i (&wf)[RW], const v4i (&af)[MT], v4i (&acc)[RW][MT]) {
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[i], af[j], acc[i][j], 0, 0, 0);
}

// ---------------------------------------------------------------------------------------
// Weight fragments of the streaming kernels, by weight layout WL:
//   0  row-major int8 [N, K], read as 16 rows x 64 bytes per instruction (16 bytes per lane)
//   1  packed int8 MFMA fragments, 1 KB per (64-byte K step, 16-row tile)
//   2  packed INT4 (W4A8): 512 bytes per (K step, tile), 8 bytes per lane.  Lane l holds row
//      16t + l%16; byte i (0..3) of its dword d carries, as two's-complement nibbles, the
//      weights at K offset 16*(l/16) + 8d + i (low nibble) and 16*(l/16) + 8d + 4 + i (high).
// ---------------------------------------------------------------------------------------
template <int WL> struct W8A8WFragT { using type = v4i; };
template <> struct W8A8WFragT<2> { using type = v2i; };
template <int WL> using W8A8WFrag = typename W8A8WFragT<WL>::type;
template <int WL> struct W8A8WFragBytes { static constexpr uint32_t value = WL == 2 ? 512u : 1024u; };

template <int WL>
__device__ __forceinline__ W8A8WFrag<WL> w8a8_wload(rsrc_t rs, uint32_t off) {
  if constexpr (WL == 2) {
    return __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 2));
  } else {
    return __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 2);
  }
}

// The MFMA A operand of a weight fragment.  An INT4 fragment expands to 16 int8 values that
// hold 16 * q: the nibble is moved to the top of its byte (low nibbles by a 4-bit shift), and
// the byte read as int8 is then 16 times the two's-complement nibble, with no carries between
// bytes.  Products and sums are therefore exactly 16 times the W4A8 ones (|16 * sum| stays
// below 2^31 for K <= 131072) and w8a8_unscale16 restores them with an exact shift.
__device__ __forceinline__ v4i w8a8_wop(v4i w) { return w; }
__device__ __forceinline__ v4i w8a8_wop(v2i w) {
  const uint32_t d0 = (uint32_t)w.x, d1 = (uint32_t)w.y;
  return v4i{(int)((d0 << 4) & 0xF0F0F0F0u), (int)(d0 & 0xF0F0F0F0u),
             (int)((d1 << 4) & 0xF0F0F0F0u), (int)(d1 & 0xF0F0F0F0u)};
}

template <int RW, int MT>
__device__ __forceinline__ void w8a8_unscale16(v4i (&acc)[RW][MT]) {
#pragma unroll
  for (int a = 0; a < RW; ++a)
#pragma unroll
    for (int u = 0; u < MT; ++u) acc[a][u] = acc[a][u] >> 4;  // every sum is a multiple of 16
}

// Epilogue for 4 consecutive output channels of one token row, with the token scale `a` and
// the channel scales `w` already in registers (entries past N are not stored).
// The fp16 outputs of 4 INT32 sums: each value is rounded to fp32 after `* a`, again after
// `* w`, and then to fp16 (RNE), as in the reference (f32_opaque keeps the compiler from
// fusing the last multiply into the fp16 conversion).
__device__ __forceinline__ v4h w8a8_cvt4(v4i s, float a, const float (&w)[4]) {
  v4h o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = (_Float16)f32_opaque(((float)s[i] * a) * w[i]);
  return o;
}
__device__ __forceinline__ void w8a8_store4s(const W8A8Params& p, int m, int n, v4i s, float a, const float (&w)[4]) {
  __half* dst = p.C + (int64_t)m * p.ldc + n;
  const v4h o = w8a8_cvt4(s, a, w);
  if (p.vec_store && n + 3 < p.N) {
    *reinterpret_cast<v4h*>(dst) = o;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (n + i < p.N) reinterpret_cast<_Float16*>(dst)[i] = o[i];
  }
}

// Epilogue for 4 consecutive output channels of one token row (scales read here).
__device__ __forceinline__ void w8a8_store4(const W8A8Params& p, int m, int n, v4i s) {
  float w[4];
  if (n + 3 < p.N) {
    const v4f q = *reinterpret_cast<const v4f*>(p.sw + n);
    w[0] = q.x; w[1] = q.y; w[2] = q.z; w[3] = q.w;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = n + i < p.N ? p.sw[n + i] : 0.f;
  }
  w8a8_store4s(p, m, n, s, p.sa[m], w);
}

// The epilogue scales of one lane's outputs, fetched before the main loop so that the
// epilogue of a weight-streaming kernel does not begin with one more memory round trip:
// sa of token rows m0 + 16u + r (u < MT) and sw of channels n0 + 16t + 4g .. + 3 (t < RW),
// lane = 16g + r.  Entries past M or N, and every entry of lanes with `use` false, are
// range-checked buffer reads that return zero without touching memory; the loads carry no
// control flow, so they do not disturb the compile-time wait counts that follow.
template <int MT, int RW>
struct W8A8EpiScales {
  float a[MT];
  float w[RW][4];
  __device__ __forceinline__ void load(const W8A8Params& p, int M, int m0, int n0, bool use) {
    const int lane = lane_id(), g = lane >> 4, r = lane & 15;
    const rsrc_t ars = make_rsrc(p.sa, (uint32_t)max(M, 0) * 4u);
    const rsrc_t wrs = make_rsrc(p.sw, (uint32_t)p.N * 4u);
#pragma unroll
    for (int u = 0; u < MT; ++u) {
      const int m = m0 + 16 * u + r;
      a[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ars, oob_unless(use & (m < M), (uint32_t)m * 4u), 0, 0));
    }
#pragma unroll
    for (int t = 0; t < RW; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = n0 + 16 * t + 4 * g + i;
        w[t][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wrs, oob_unless(use & (n < p.N), (uint32_t)n * 4u), 0, 0));
      }
  }
};

// Split-K hand-off of a workgroup's INT32 tile [BM][BN] (row = token), 16 bytes per lane.
// Partials of tile cidx live at p.partials + cidx * splits * BM * BN, split-major.
template <int BM, int BN>
__device__ __forceinline__ rsrc_t w8a8_partials_rsrc(const W8A8Params& p, int cidx) {
  return make_rsrc(p.partials + (int64_t)cidx * p.splits * (BM * BN), (uint32_t)(p.splits * BM * BN * 4));
}
// Publish the quad of channels nl..nl+3 (tile-local) of token row ml (tile-local).
template <int BM, int BN>
__device__ __forceinline__ void w8a8_publish_quad(rsrc_t prs, int split, int ml, int nl, v4i v) {
  publish16(prs, (uint32_t)(((split * BM + ml) * BN + nl) * 4), v);
}
// Called by every thread after its publishes: the last workgroup of the tile to arrive sums
// the splits and applies the epilogue.  Thread t owns quads t, t + NT, ...; the partials of up
// to QG quads x SB splits are loaded together, so the sum costs one memory round trip per
// group instead of one per quad (INT32 sums are order independent).  The first group's scales
// are loaded before the arrival, in flight with the stores of the partial tiles.
template <int BM, int BN, int NT>
__device__ __forceinline__ void w8a8_splitk_finish(const W8A8Params& p, rsrc_t prs, int cidx, int m0, int nbase,
                                                   int M, int* s_last) {
  constexpr int QUADS = BM * BN / 4;
  constexpr int QPT = (QUADS + NT - 1) / NT;                   // quads per thread
  // Up to 8 quads per thread are summed in one round of loads (up to 32 loads in flight);
  // the deepest tiles, whose main loops need every register, take 4 quads per round.
  constexpr int QG = QPT <= 8 ? QPT : 4;                       // quads summed together
  constexpr int SB = (QPT <= 8 ? 32 : 16) / QG > 8 ? 8 : (QPT <= 8 ? 32 : 16) / QG;  // splits loaded together
  int ml[QG], nl[QG];
  bool ok[QG];
  float a[QG], w[QG][4];
  auto prepare = [&](int g0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < QG; ++i) {
      const int q = (int)threadIdx.x + (g0 + i) * NT;
      ml[i] = q / (BN / 4);
      nl[i] = (q % (BN / 4)) * 4;
      const int m = m0 + ml[i], n = nbase + nl[i];
      ok[i] = (g0 + i < QPT) & (q < QUADS) & (m < M) & (n < p.N);
      // Indices clamped into range (the values of lanes that do not store are unused), so
      // the loads need no branch and no extra buffer descriptors.
      a[i] = p.sa[ok[i] ? m : m0];
#pragma unroll
      for (int c = 0; c < 4; ++c) w[i][c] = p.sw[min(ok[i] ? n + c : nbase, p.N - 1)];
    }
  };
  prepare(0);
  if (!arrive_last(p.counters + cidx, p.splits, s_last, p.tl, p.tl_cap)) return;
#pragma unroll
  for (int g0 = 0; g0 < QPT; g0 += QG) {
    if (g0 > 0) prepare(g0);
    v4i s[QG];
#pragma unroll
    for (int i = 0; i < QG; ++i) s[i] = v4i{0, 0, 0, 0};
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
        for (int u = 0; u < SB; ++u) s[i] += t[i][u];
    }
    if (g0 == 0) tl_mark(p.tl, p.tl_cap, 7);  // diagnostics build: first group of partials summed
#pragma unroll
    for (int i = 0; i < QG; ++i)
      if (ok[i]) w8a8_store4s(p, m0 + ml[i], nbase + nl[i], s[i], a[i], w[i]);
  }
}

template <int MT, int RW, int VEC>
__global__ __launch_bounds__(256) void w8a8_kernel(W8A8Params p) {
  constexpr int BM = MT * 16, BN = RW * 16, U = W8A8Unroll<MT, RW>::value;
  constexpr int LDW = BN + kW8A8Pad;  // LDS row pitch in int32
  extern __shared__ int32_t smem[];

  const int nw = blockDim.x / kWave;
  int mc, unit;
  if (!chunked_unit(p.m_chunks, p.n_tiles * p.splits, mc, unit)) return;
  const int split = unit % p.splits;
  const int tile = unit / p.splits;

  int M = p.M;
  if (p.plan != nullptr) M = min(max(p.plan[0], 0), p.m_grid);
  M = uniform(M);
  const int m0 = mc * BM;
  if (m0 >= M) return;  // plan guard: inactive M-chunk, nothing read or written

  const int n0 = tile * BN;
  const int kb = split * p.k_range;
  const int ke = min(p.K, kb + p.k_range);
  const int lane = lane_id(), w = wave_id(), g = lane >> 4, r = lane & 15;

  // Buffer resources over this workgroup's slabs: rows past N (or past the active M) and
  // K positions past the split read as zero, with no branches around the loads.
  const int n_rows = min(BN, p.N - n0), m_rows = min(BM, M - m0);
  const rsrc_t wsrc = make_rsrc(p.W + (int64_t)n0 * p.ldw, (uint32_t)((n_rows - 1) * p.ldw + p.K));
  const rsrc_t asrc = make_rsrc(p.A + (int64_t)m0 * p.lda, (uint32_t)((m_rows - 1) * p.lda + p.K));
  uint32_t woff[RW], aoff[MT];
#pragma unroll
  for (int i = 0; i < RW; ++i) woff[i] = (i * 16 + r < n_rows) ? (uint32_t)((i * 16 + r) * p.ldw) : kOOB;
#pragma unroll
  for (int j = 0; j < MT; ++j) aoff[j] = (j * 16 + r < m_rows) ? (uint32_t)((j * 16 + r) * p.lda) : kOOB;

  v4i acc[RW][MT];
#pragma unroll
  for (int i = 0; i < RW; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  // This wave's K steps: kb + (w + t*nw)*64 for t = 0..nsteps-1, batched U at a time and
  // double-buffered in registers (loads of batch b+1 are in flight during batch b's MFMAs).
  const int stride = nw * 64;
  const int k_first = kb + w * 64 + g * 16;
  const int nsteps = (kb + w * 64 < ke) ? (ke - (kb + w * 64) + stride - 1) / stride : 0;
  const int nbatch = (nsteps + U - 1) / U;

  v4i wa[U][RW], aa[U][MT], wb[U][RW], ab[U][MT];
  auto load_batch = [&](int b, v4i (&wv)[U][RW], v4i (&av)[U][MT]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = k_first + (b * U + u) * stride;
#pragma unroll
      for (int i = 0; i < RW; ++i) wv[u][i] = bload16<VEC>(wsrc, woff[i], k, ke);
#pragma unroll
      for (int j = 0; j < MT; ++j) av[u][j] = bload16<VEC>(asrc, aoff[j], k, ke);
    }
  };
  auto mma_batch = [&](v4i (&wv)[U][RW], v4i (&av)[U][MT]) {
#pragma unroll
    for (int u = 0; u < U; ++u) w8a8_mma_step<MT, RW>(wv[u], av[u], acc);
  };

  // The loop body has no branches: batches past this wave's range (the odd tail and the
  // prefetch beyond the end) read zeros through the range check and add nothing, so the
  // compiler can keep exactly one batch of loads in flight behind each batch of MFMAs.
  load_batch(0, wa, aa);
  for (int b = 0; b < nbatch; b += 2) {
    load_batch(b + 1, wb, ab);
    mma_batch(wa, aa);
    load_batch(b + 2, wa, aa);
    mma_batch(wb, ab);
  }

  // Cross-wave reduction through one LDS slice [BM][LDW]: waves nw-1 .. 1 each deposit their
  // accumulators in turn and wave 0 adds them into its registers.  Lane (r, g) of 16x16 block
  // (i, j) holds channels n = i*16 + 4g + {0..3} of token m = j*16 + r.
  for (int src = nw - 1; src >= 1; --src) {
    if (w == src) {
#pragma unroll
      for (int i = 0; i < RW; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j)
          *reinterpret_cast<v4i*>(smem + (j * 16 + r) * LDW + i * 16 + 4 * g) = acc[i][j];
    }
    __syncthreads();
    if (w == 0) {
#pragma unroll
      for (int i = 0; i < RW; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j)
          acc[i][j] += *reinterpret_cast<const v4i*>(smem + (j * 16 + r) * LDW + i * 16 + 4 * g);
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

  // Split-K fix-up: every split publishes its INT32 tile ([BM][BN], row = token); the last
  // workgroup of this (M-chunk, N-tile) to arrive sums all splits and applies the epilogue.
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
