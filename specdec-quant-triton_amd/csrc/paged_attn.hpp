// INT8 paged-KV verification attention for gfx950.
//
// Computes, for every active sequence b, KV head h, query token i (of the q_len appended to
// the context) and query head of the GQA group, the reference's kernels.py:178-236:
//   s_t = (q . k_t) * ks_t * sm_scale   for t <= L - q_len + i   (causal on absolute position)
//   p_t = softmax_t(s)                  (online, rows with no visible key give 0)
//   o   = sum_t fp16(p_t * vs_t) * v_t  (the V scale is folded into P before the PV product)
// K/V are int8 [pages, PAGE, H_KV, D] reached through a block table; scales are fp16 or fp32.
//
// MI355X schedule:
//  * One workgroup = (KV split, KV head, query chunk of QPP tokens, sequence).  A split is 512
//    tokens, or a multiple of 512 for block tables longer than 64 x 512 tokens.
//    The QPP * G query rows sharing the KV head are packed into RB 16-row blocks, so a fused
//    verification program reads each K/V byte once for all (k+1) * G rows.
//  * The four waves take interleaved 32-token chunks of the split (chunk c of the split goes
//    to wave c % 4) and stream them through a two-deep register pipeline: the K rows, V rows
//    and scales of the wave's next chunk are in flight while the current one is multiplied.
//    Every lane loads 16-byte pieces: a K row is 4 lanes x 32 B, a V row 8 lanes x 16 B, one
//    lane per token for each scale, all through the block table (one 16-token page sub-tile
//    per page lookup).  Loads are never branched around: tokens past the program's last
//    visible key read a valid dummy address (finite int8 whose P is 0).
//  * S^T = K . Q^T on v_mfma_f32_16x16x32_f16 with K as the A-operand (int8 converted to fp16
//    in registers by exponent injection).  The result lands with the query row in lane % 16,
//    which is exactly the B-operand layout of the next product, so P never moves between
//    lanes.  The scales of the chunk pass through a small wave-private LDS staging area so a
//    lane reads the 4 consecutive tokens it needs with one 16-byte LDS read.
//  * O^T = V^T . P^T with V^T as the A-operand.  V rows are transposed through a wave-private
//    LDS tile (4x4 byte transposes with v_perm, dword writes, two dword reads per operand).
//    The O accumulator then also has the query row in lane % 16, so the online-softmax
//    rescale is lane local.
//  * The waves merge in a fixed order through LDS; splits merge in split order through the
//    workspace (16-byte hand-offs, last workgroup to arrive).  The split boundaries and the
//    chunk-to-wave assignment are fixed token positions, so a row's result is bit-identical
//    whether it is computed by a QPP=1 or a fused program, eagerly or from a plan-mode graph.
//  * Plan mode reads (n_seqs, q_len) from plan[0..1]; programs for inactive sequences or
//    query slots return before any load or store.
#pragma once
#include "common.hpp"

namespace specq {

struct AttnParams {
  const _Float16* q; int64_t s_qb, s_qt, s_qh;
  const int8_t* kc; const int8_t* vc; int64_t s_kp, s_ko, s_kh;
  const void* ks; const void* vs; int64_t s_sp, s_so, s_sh;
  const int32_t* bt; int64_t s_bt; int max_pages;
  const int32_t* ctx_len;
  _Float16* out; int64_t s_ob, s_ot, s_oh;
  const int32_t* plan;
  int B_grid, n_seqs, q_len, ql_grid;
  int G, QPP, n_qc, H_KV, PAGE;
  int n_splits;        // splits the grid covers per program
  int split_sub;       // 512-token sub-splits per split (longer contexts keep n_splits <= 64)
  float scale_log2;    // sm_scale * log2(e)
  float* part;         // [progs][n_splits][rows][D] unnormalised O, then [progs][n_splits][rows][2] (m, l)
  int32_t* counters;   // [progs]
};

constexpr int kAttnSplitTokens = 512;  // tokens per workgroup (KV split)
constexpr int kAttnChunk = 32;         // tokens per wave iteration
constexpr int kAttnWaves = 4;
constexpr int kAttnVtPitch = 36;       // bytes per d-row of the transposed V tile (32 tokens + pad)
constexpr int kAttnMergeMax = 64;      // most splits one program merges (fits the o_lds tile for D >= 64)

template <typename ST>
__device__ __forceinline__ float load_scale(const void* base, int64_t idx) {
  return (float)reinterpret_cast<const ST*>(base)[idx];
}

// 4x4 byte transpose: x[j] holds 4 consecutive d bytes of token j; y[d] gets the 4 token bytes of d.
__device__ __forceinline__ void transpose4x4(const uint32_t (&x)[4], uint32_t (&y)[4]) {
  uint32_t t0 = __builtin_amdgcn_perm(x[1], x[0], 0x05010400u);
  uint32_t t1 = __builtin_amdgcn_perm(x[1], x[0], 0x07030602u);
  uint32_t t2 = __builtin_amdgcn_perm(x[3], x[2], 0x05010400u);
  uint32_t t3 = __builtin_amdgcn_perm(x[3], x[2], 0x07030602u);
  y[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
  y[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
  y[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
  y[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

template <int D, int RB, typename ST>
__global__ __launch_bounds__(256) void paged_attn_kernel(AttnParams p) {
  constexpr int NU = D / 32;          // MFMA K-steps over the head dimension
  constexpr int ND = D / 16;          // 16-wide d blocks of the output
  constexpr int DS = D / 4;           // head-dim bytes a lane holds per token (K) or row (Q)
  constexpr int DB = D / 8;           // V bytes per lane per token
  constexpr int ROWS = RB * 16;
  constexpr int IT = kAttnSplitTokens / kAttnChunk / kAttnWaves;  // chunks per wave
  constexpr int KV4 = D / 64;         // 16-byte K pieces per lane per 16-token sub-tile
  constexpr int VW = D / 32;          // dwords per lane per V row piece
  __shared__ __attribute__((aligned(16))) uint8_t vt_lds[kAttnWaves][D * kAttnVtPitch];
  __shared__ __attribute__((aligned(16))) float sc_lds[kAttnWaves][64];
  __shared__ float ml_lds[kAttnWaves][2][ROWS];
  __shared__ __attribute__((aligned(16))) float o_lds[ROWS][D + 4];
  // Q fragments in MFMA B-operand order: [rb][u][lane] of 16 bytes (zero for padding rows).
  __shared__ __attribute__((aligned(16))) v8h q_lds[RB][NU][64];
  __shared__ int s_last;

  const int split = blockIdx.x;
  const int kvh = blockIdx.y / p.n_qc, qc = blockIdx.y % p.n_qc;
  const int b = blockIdx.z;
  int n_seqs = p.n_seqs, q_len = p.q_len;
  if (p.plan != nullptr) {
    n_seqs = min(max(p.plan[0], 0), p.B_grid);
    q_len = min(max(p.plan[1], 0), p.ql_grid);
  }
  n_seqs = uniform(n_seqs);
  q_len = uniform(q_len);
  if (b >= n_seqs || qc * p.QPP >= q_len) return;
  // The block table holds max_pages pages: never look past them.
  const int L = uniform(min(p.ctx_len[b], p.max_pages * p.PAGE));
  const int kv_end = L - q_len + min(qc * p.QPP + p.QPP, q_len);
  // Split 0 always runs, so rows with no visible key still get their zero output.
  const int split_tokens = kAttnSplitTokens * p.split_sub;
  if (split > 0 && split * split_tokens >= kv_end) return;
  const int n_active = kv_end > split_tokens ? (kv_end + split_tokens - 1) / split_tokens : 1;

  const int lane = lane_id(), w = wave_id(), g = lane >> 4, r = lane & 15;
  const int G = p.G;

  // Query rows held by this lane (one per row block): row = rb*16 + r.  Their B-operand
  // fragments go to LDS once (each wave writes its share of the row blocks) and are read back
  // per MFMA, which leaves registers for a three-chunk load pipeline.
  int qpos[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = rb * 16 + r;
    const int qi = qc * p.QPP + row / G;
    const bool valid = (row < p.QPP * G) && (qi < q_len);
    qpos[rb] = valid ? (L - q_len + qi) : -1;
  }

  float m_run[RB], l_run[RB];
  v4f acc[RB][ND];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m_run[rb] = -INFINITY;
    l_run[rb] = 0.f;
#pragma unroll
    for (int db = 0; db < ND; ++db) acc[rb][db] = v4f{0.f, 0.f, 0.f, 0.f};
  }

  uint8_t* vt = vt_lds[w];
  float* scw = sc_lds[w];
  const int64_t kv_head_off = (int64_t)kvh * p.s_kh;
  const int64_t sc_head_off = (int64_t)kvh * p.s_sh;
  const int32_t* bt_row = p.bt + (int64_t)b * p.s_bt;
  const int PAGE = p.PAGE;

  // ---- Chunk loads.  Chunk `it` of this wave starts at token t0(it); its two 16-token
  // sub-tiles each lie in one page.  Masked tokens (at or past kv_end) read the first bytes of
  // the cache instead: their int8 K/V are finite, their scores are masked to -inf and their P
  // is 0, so they add nothing; their scales are zeroed.
  int sub_base = split * split_tokens;  // first token of the current 512-token sub-split
  auto chunk_t0 = [&](int it) { return sub_base + (it * kAttnWaves + w) * kAttnChunk; };
  // Register double buffer of the raw chunk bytes: K pieces, V pieces, one scale per lane
  // (lane l < 32: ks of token l; lane >= 32: vs of token l - 32).
  constexpr int NB = 2;  // chunks in the register pipeline
  v4i kbuf[NB][2][KV4];
  uint32_t vbuf[NB][4][VW];
  float sbuf[NB];
  // Pages of the wave's 2 * IT sub-tiles in the current 512-token sub-split, looked up together
  // at its start (one block-table round trip instead of one per chunk).
  int pages[IT][2];
  auto lookup_pages = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int it = 0; it < IT; ++it)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int ts = chunk_t0(it) + 16 * j;
        pages[it][j] = ts < kv_end ? bt_row[ts / PAGE] : 0;
      }
  };
  auto load_chunk = [&](auto bic, auto itc) __attribute__((always_inline)) {
    constexpr int bi = decltype(bic)::value;
    constexpr int it = decltype(itc)::value;
    const int t0 = chunk_t0(it);
    int64_t pbase[2];  // element offset of (page, token 0 of the sub-tile, this KV head) in the cache
    int64_t sbase[2];  // element offset of the sub-tile's first scale
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ts = t0 + 16 * j;
      pbase[j] = (int64_t)pages[it][j] * p.s_kp + (int64_t)(ts % PAGE) * p.s_ko + kv_head_off;
      sbase[j] = (int64_t)pages[it][j] * p.s_sp + (int64_t)(ts % PAGE) * p.s_so + sc_head_off;
    }
    // K: lane (r, g) holds bytes [DS*g, DS*g + DS) of token 16j + r.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const bool ok = t0 + 16 * j + r < kv_end;
      const int8_t* src = p.kc + (ok ? pbase[j] + (int64_t)r * p.s_ko + DS * g : 0);
#pragma unroll
      for (int h = 0; h < KV4; ++h) kbuf[bi][j][h] = *reinterpret_cast<const v4i*>(src + 16 * h);
    }
    // V: lane (tq = lane / 8, dq = lane % 8) holds DB bytes at d = DB*dq of tokens 4tq .. 4tq+3.
    {
      const int tq = lane >> 3, dq = lane & 7, j = tq >> 2;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tl = 4 * (tq & 3) + i;  // token within sub-tile j
        const bool ok = t0 + 16 * j + tl < kv_end;
        const int8_t* src = p.vc + (ok ? pbase[j] + (int64_t)tl * p.s_ko + DB * dq : 0);
        if constexpr (VW == 4) {
          const v4i x = *reinterpret_cast<const v4i*>(src);
          vbuf[bi][i][0] = (uint32_t)x.x; vbuf[bi][i][1] = (uint32_t)x.y;
          vbuf[bi][i][2] = (uint32_t)x.z; vbuf[bi][i][3] = (uint32_t)x.w;
        } else {
          const v2i x = *reinterpret_cast<const v2i*>(src);
          vbuf[bi][i][0] = (uint32_t)x.x; vbuf[bi][i][1] = (uint32_t)x.y;
        }
      }
    }
    // Scales: lane l holds ks (l < 32) or vs (l >= 32) of token l % 32.
    {
      const int tl = lane & 31, j = tl >> 4;
      const bool ok = t0 + tl < kv_end;
      const int64_t si = ok ? sbase[j] + (int64_t)(tl & 15) * p.s_so : 0;
      const float x = load_scale<ST>(lane < 32 ? p.ks : p.vs, si);
      sbuf[bi] = ok ? x : 0.f;
    }
  };

  // ---- One chunk: stage V^T and the scales in LDS, S^T, online softmax, O^T += V^T . P^T.
  auto compute_chunk = [&](auto bic, int it) __attribute__((always_inline)) {
    constexpr int bi = decltype(bic)::value;
    const int t0 = chunk_t0(it);
    // Stage: Vt[d][token] for d in [DB*dq, DB*dq + DB), tokens 4tq..4tq+3; the 64 scales.
    {
      const int tq = lane >> 3, dq = lane & 7;
#pragma unroll
      for (int cc = 0; cc < DB / 4; ++cc) {
        uint32_t x[4] = {vbuf[bi][0][cc], vbuf[bi][1][cc], vbuf[bi][2][cc], vbuf[bi][3][cc]};
        uint32_t y[4];
        transpose4x4(x, y);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          *reinterpret_cast<uint32_t*>(vt + (DB * dq + 4 * cc + e) * kAttnVtPitch + 4 * tq) = y[e];
      }
      scw[lane] = sbuf[bi];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // Scales of the lane's tokens 16j + 4g + i: ks at [0, 32), vs at [32, 64).
    v4f ksc[2], vsc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      ksc[j] = *reinterpret_cast<const v4f*>(scw + 16 * j + 4 * g);
      vsc[j] = *reinterpret_cast<const v4f*>(scw + 32 + 16 * j + 4 * g);
    }
    // K fragment u of sub-tile j (8 int8 -> fp16), converted where it is used.
    auto kfrag = [&](int j, int u) __attribute__((always_inline)) {
      const v4i& x = kbuf[bi][j][u >> 1];
      return (u & 1) ? i8x8_to_h8((uint32_t)x.z, (uint32_t)x.w) : i8x8_to_h8((uint32_t)x.x, (uint32_t)x.y);
    };

    // Every row of the program sees every token of the chunk: no causal mask needed.
    const bool full = t0 + kAttnChunk - 1 <= L - q_len + qc * p.QPP;
    v8h pf[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float s[2][4];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        v4f cs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < NU; ++u) cs = __builtin_amdgcn_mfma_f32_16x16x32_f16(kfrag(j, u), q_lds[rb][u][lane], cs, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = t0 + 16 * j + 4 * g + i;
          const float v = cs[i] * (ksc[j][i] * p.scale_log2);
          s[j][i] = (full || t <= qpos[rb]) ? v : -INFINITY;
        }
      }
      float cmax = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                         fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
      cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
      cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
      const float m_new = fmaxf(m_run[rb], cmax);
      const float m_safe = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = fast_exp2(m_run[rb] - m_safe);
      float psum = 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pv = fast_exp2(s[j][i] - m_safe);
          psum += pv;
          pf[rb][4 * j + i] = (_Float16)(pv * vsc[j][i]);
        }
      l_run[rb] = l_run[rb] * alpha + psum;
      // alpha is exactly 1 for every row whose running max did not grow, so the O rescale is
      // skipped (bit-identically) unless some row of the wave's block grew, which after the
      // first chunks is rare; the accumulators then stay in the MFMA's registers.
      const bool grew = m_new > m_run[rb];
      m_run[rb] = m_new;
      if (__builtin_amdgcn_ballot_w64(grew) != 0) {
#pragma unroll
        for (int db = 0; db < ND; ++db) acc[rb][db] *= alpha;
      }
    }

    // O^T += V^T . P^T  (A-operand: lane (d, g) holds tokens {4g..4g+3, 16+4g..16+4g+3} of d)
#pragma unroll
    for (int db = 0; db < ND; ++db) {
      const uint8_t* vrow = vt + (db * 16 + r) * kAttnVtPitch;
      const uint32_t v0 = *reinterpret_cast<const uint32_t*>(vrow + 4 * g);
      const uint32_t v1 = *reinterpret_cast<const uint32_t*>(vrow + 16 + 4 * g);
      const v8h vf = i8x8_to_h8(v0, v1);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        acc[rb][db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[rb], acc[rb][db], 0, 0, 0);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  // Chunk it + 1 is in flight while chunk it is multiplied; the first sub-split's
  // page lookups and first loads are issued before the Q fragments are staged, so those
  // memory round trips overlap.
  // Q fragments: thread t stages fragments t, t + 256, ... of [rb][u][lane].
  constexpr int QF = (RB * NU * 64 + 255) / 256;
  auto q_frag_valid = [&](int f) {
    const int row = (f / (NU * 64)) * 16 + (f % 64 & 15);
    return f < RB * NU * 64 && (row < p.QPP * G) && (qc * p.QPP + row / G < q_len);
  };
  auto q_frag_src = [&](int f) -> const _Float16* {  // a valid fragment's 8 halves
    const int rb = f / (NU * 64), u = (f / 64) % NU, ln = f % 64;
    const int row = rb * 16 + (ln & 15);
    const int qi = qc * p.QPP + row / G;
    const int head = kvh * G + row % G;
    return p.q + (int64_t)b * p.s_qb + (int64_t)qi * p.s_qt + (int64_t)head * p.s_qh + DS * (ln >> 4) + 8 * u;
  };
  bool staged = false;
  for (int sub = 0; sub < p.split_sub && sub_base < kv_end; ++sub, sub_base += kAttnSplitTokens) {
    lookup_pages();
    v8h qtmp[QF];
    if (!staged) {
#pragma unroll
      for (int i = 0; i < QF; ++i) {
        const int f = threadIdx.x + 256 * i;
        const bool ok = q_frag_valid(f);
        const v8h x = *reinterpret_cast<const v8h*>(ok ? q_frag_src(f) : p.q);
        qtmp[i] = ok ? x : v8h{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
    static_for<0, NB - 1>([&](auto ic) __attribute__((always_inline)) {
      constexpr int i = decltype(ic)::value;
      if constexpr (i < IT) load_chunk(std::integral_constant<int, i>{}, std::integral_constant<int, i>{});
    });
    if (!staged) {
      // The Q fragments go to LDS while the first chunks stay in flight (the barrier waits
      // for LDS only).
#pragma unroll
      for (int i = 0; i < QF; ++i) {
        const int f = threadIdx.x + 256 * i;
        if (f < RB * NU * 64) (&q_lds[0][0][0])[f] = qtmp[i];
      }
      wg_barrier_lds();
      staged = true;
    }
    static_for<0, IT>([&](auto itc) __attribute__((always_inline)) {
      constexpr int it = decltype(itc)::value;
      if constexpr (it + NB - 1 < IT)
        load_chunk(std::integral_constant<int, (it + NB - 1) % NB>{}, std::integral_constant<int, it + NB - 1>{});
      if (chunk_t0(it) < kv_end) compute_chunk(std::integral_constant<int, it % NB>{}, it);
    });
  }

  // ---- Merge the four waves in a fixed order.
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    float lr = l_run[rb];
    lr += __shfl_xor(lr, 16);
    lr += __shfl_xor(lr, 32);
    if (g == 0) {
      ml_lds[w][0][rb * 16 + r] = m_run[rb];
      ml_lds[w][1][rb * 16 + r] = lr;
    }
  }
  __syncthreads();
  float wscale[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = rb * 16 + r;
    float mx = ml_lds[0][0][row];
#pragma unroll
    for (int ww = 1; ww < kAttnWaves; ++ww) mx = fmaxf(mx, ml_lds[ww][0][row]);
    const float ms = (mx == -INFINITY) ? 0.f : mx;
    wscale[rb] = fast_exp2(m_run[rb] - ms);
  }
  for (int ww = 0; ww < kAttnWaves; ++ww) {
    if (w == ww) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int db = 0; db < ND; ++db) {
          v4f* dst = reinterpret_cast<v4f*>(&o_lds[rb * 16 + r][db * 16 + 4 * g]);
          const v4f v = acc[rb][db] * wscale[rb];
          *dst = (ww == 0) ? v : (*dst + v);
        }
    }
    __syncthreads();
  }
  // Row statistics of the workgroup: max and scaled sum, in wave order.
  if (threadIdx.x < ROWS) {
    const int row = threadIdx.x;
    float mx = ml_lds[0][0][row];
    for (int ww = 1; ww < kAttnWaves; ++ww) mx = fmaxf(mx, ml_lds[ww][0][row]);
    const float ms = (mx == -INFINITY) ? 0.f : mx;
    float ls = 0.f;
    for (int ww = 0; ww < kAttnWaves; ++ww) ls += fast_exp2(ml_lds[ww][0][row] - ms) * ml_lds[ww][1][row];
    ml_lds[0][0][row] = mx;
    ml_lds[0][1][row] = ls;
  }
  __syncthreads();

  const int prog = (b * p.H_KV + kvh) * p.n_qc + qc;
  constexpr int DCH = D / 8;  // 8-element chunks per row
  if (n_active == 1) {
    for (int e = threadIdx.x; e < ROWS * DCH; e += blockDim.x) {
      const int row = e / DCH, d0 = (e % DCH) * 8;
      const int qi = qc * p.QPP + row / G;
      if (!(row < p.QPP * G && qi < q_len)) continue;
      const int head = kvh * G + row % G;
      const float l = ml_lds[0][1][row];
      const float inv = (l == 0.f) ? 0.f : 1.f / l;
      v8h o;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (_Float16)(o_lds[row][d0 + i] * inv);
      *reinterpret_cast<v8h*>(p.out + (int64_t)b * p.s_ob + (int64_t)qi * p.s_ot + (int64_t)head * p.s_oh + d0) = o;
    }
    return;
  }

  // ---- Cross-split merge: publish this split (16 bytes per lane), the last to arrive combines
  // the splits in split order.
  const int64_t prog_base = (int64_t)prog * p.n_splits;
  const int64_t n_o = (int64_t)gridDim.y * gridDim.z * p.n_splits * ROWS * D;  // floats of the O region
  const rsrc_t ors = make_rsrc(p.part + prog_base * ROWS * D, (uint32_t)(p.n_splits * ROWS * D * 4));
  float* mlpart = p.part + n_o;
  for (int e = threadIdx.x; e < ROWS * D / 4; e += blockDim.x) {
    const int row = e / (D / 4), d = (e % (D / 4)) * 4;
    const v4f v = *reinterpret_cast<const v4f*>(&o_lds[row][d]);
    publish16(ors, (uint32_t)(((split * ROWS + row) * D + d) * 4), __builtin_bit_cast(v4i, v));
  }
  if (threadIdx.x < ROWS) {
    float* mlp = mlpart + ((prog_base + split) * ROWS + threadIdx.x) * 2;
    publish(mlp, ml_lds[0][0][threadIdx.x]);
    publish(mlp + 1, ml_lds[0][1][threadIdx.x]);
  }
  if (!arrive_last(p.counters + prog, n_active, &s_last)) return;
  // Row weights of the splits, exp2(m_s - max) / l (l summed in split order), kept in the
  // o_lds tile (already published).  Up to 16 splits the (m, l) pairs are loaded once, all in
  // flight together; more splits take a second pass.
  constexpr int kMergeBatch = 16;
  if (threadIdx.x < ROWS) {
    const int row = threadIdx.x;
    float* wt = &o_lds[row][0];
    auto ml_at = [&](int sp) { return mlpart + ((prog_base + (sp < n_active ? sp : 0)) * ROWS + row) * 2; };
    float mv[kMergeBatch], lv[kMergeBatch];
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      mv[u] = collect(ml_at(u));
      lv[u] = collect(ml_at(u) + 1);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u)
      if (u < n_active) mx = fmaxf(mx, mv[u]);
    for (int sp = kMergeBatch; sp < n_active; ++sp) mx = fmaxf(mx, collect(ml_at(sp)));
    const float mxs = (mx == -INFINITY) ? 0.f : mx;
    float l = 0.f;
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u)
      if (u < n_active) {
        const float wgt = fast_exp2(mv[u] - mxs);
        wt[u] = wgt;
        const float lw = wgt * lv[u];
        l = (u == 0) ? lw : l + lw;
      }
    for (int sp = kMergeBatch; sp < n_active; ++sp) {
      const float wgt = fast_exp2(collect(ml_at(sp)) - mxs);
      wt[sp] = wgt;
      l += wgt * collect(ml_at(sp) + 1);
    }
    const float inv = (l == 0.f) ? 0.f : 1.f / l;
    for (int sp = 0; sp < n_active; ++sp) wt[sp] *= inv;
  }
  __syncthreads();
  // O rows: sum over splits in split order of weight * partial O.  Thread t owns the 4-column
  // items t, t + 256, ...; all of its items' loads of 4 splits are in flight together.
  constexpr int QPR = D / 4;                       // 4-column items per row
  constexpr int ITEMS = (ROWS * QPR + 255) / 256;  // items per thread
  constexpr int SB = 8;                            // splits per batch
  v4f o[ITEMS];
  uint32_t ioff[ITEMS];
  bool ivalid[ITEMS];
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int e = threadIdx.x + 256 * it;
    const int row = e / QPR, d0 = (e % QPR) * 4;
    const int qi = qc * p.QPP + row / G;
    ivalid[it] = e < ROWS * QPR && row < p.QPP * G && qi < q_len;
    ioff[it] = (uint32_t)((row * D + d0) * 4);
    o[it] = v4f{0.f, 0.f, 0.f, 0.f};
  }
  for (int s0 = 0; s0 < n_active; s0 += SB) {
    v4i t[SB][ITEMS];
#pragma unroll
    for (int u = 0; u < SB; ++u)
#pragma unroll
      for (int it = 0; it < ITEMS; ++it)
        t[u][it] = collect16(ors, oob_unless(ivalid[it] && s0 + u < n_active,
                                             (uint32_t)((s0 + u) * ROWS * D * 4) + ioff[it]));
#pragma unroll
    for (int u = 0; u < SB; ++u)
#pragma unroll
      for (int it = 0; it < ITEMS; ++it)
        if (ivalid[it] && s0 + u < n_active) {
          const int e = threadIdx.x + 256 * it;
          o[it] += o_lds[e / QPR][s0 + u] * __builtin_bit_cast(v4f, t[u][it]);
        }
  }
  typedef _Float16 v4h_t __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    if (!ivalid[it]) continue;
    const int e = threadIdx.x + 256 * it;
    const int row = e / QPR, d0 = (e % QPR) * 4;
    const int qi = qc * p.QPP + row / G;
    const int head = kvh * G + row % G;
    *reinterpret_cast<v4h_t*>(p.out + (int64_t)b * p.s_ob + (int64_t)qi * p.s_ot + (int64_t)head * p.s_oh + d0) =
        v4h_t{(_Float16)o[it].x, (_Float16)o[it].y, (_Float16)o[it].z, (_Float16)o[it].w};
  }
}

}  // namespace specq
