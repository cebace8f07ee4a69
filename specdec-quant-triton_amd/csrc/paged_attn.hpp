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
//  * One workgroup = (KV split of 512 tokens, KV head, query chunk of QPP tokens, sequence).
//    The QPP * G query rows sharing the KV head are packed into RB 16-row blocks, so a fused
//    verification program reads each K/V byte once for all (k+1) * G rows.
//  * S^T = K . Q^T on v_mfma_f32_16x16x32_f16 with K as the A-operand: each lane loads 32
//    contiguous int8 bytes of one token row straight from HBM (block-table indirection per
//    16-token page) and converts them to fp16 in registers.  The result lands with the query
//    row in lane % 16, which is exactly the B-operand layout of the next product, so P never
//    moves between lanes.
//  * O^T = V^T . P^T with V^T as the A-operand.  V rows are transposed through a wave-private
//    LDS tile (4x4 byte transposes with v_perm, dword writes, two dword reads per operand).
//    The O accumulator then also has the query row in lane % 16, so the online-softmax
//    rescale is lane local.
//  * The four waves of a workgroup take interleaved 32-token chunks of its split and merge
//    in a fixed order through LDS; splits merge in split order through the workspace (last
//    workgroup to arrive).  The split boundaries are fixed token positions, so a row's result
//    is bit-identical whether it is computed by a QPP=1 or a fused program, eagerly or from
//    a plan-mode graph.
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
  float scale_log2;    // sm_scale * log2(e)
  float* part;         // [progs][n_splits][rows][D] unnormalised O, then [progs][n_splits][rows][2] (m, l)
  int32_t* counters;   // [progs]
};

constexpr int kAttnSplitTokens = 512;  // tokens per workgroup (KV split)
constexpr int kAttnChunk = 32;         // tokens per wave iteration
constexpr int kAttnWaves = 4;
constexpr int kAttnVtPitch = 36;       // bytes per d-row of the transposed V tile (32 tokens + pad)

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
  constexpr int ROWS = RB * 16;
  constexpr int CHUNKS = kAttnSplitTokens / kAttnChunk;
  __shared__ __attribute__((aligned(16))) uint8_t vt_lds[kAttnWaves][D * kAttnVtPitch];
  __shared__ float ml_lds[kAttnWaves][2][ROWS];
  __shared__ __attribute__((aligned(16))) float o_lds[ROWS][D + 4];
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
  if (split > 0 && split * kAttnSplitTokens >= kv_end) return;
  const int n_active = kv_end > kAttnSplitTokens ? (kv_end + kAttnSplitTokens - 1) / kAttnSplitTokens : 1;

  const int lane = lane_id(), w = wave_id(), g = lane >> 4, r = lane & 15;
  const int G = p.G;

  // Query rows held by this lane (one per row block): row = rb*16 + r.
  int qpos[RB];
  bool rvalid[RB];
  v8h qf[RB][NU];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = rb * 16 + r;
    const int qi = qc * p.QPP + row / G;
    const int head = kvh * G + row % G;
    rvalid[rb] = (row < p.QPP * G) && (qi < q_len);
    qpos[rb] = rvalid[rb] ? (L - q_len + qi) : -1;
    const _Float16* qrow = p.q + (int64_t)b * p.s_qb + (int64_t)qi * p.s_qt + (int64_t)head * p.s_qh + DS * g;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      if (rvalid[rb]) qf[rb][u] = *reinterpret_cast<const v8h*>(qrow + 8 * u);
      else qf[rb][u] = v8h{0, 0, 0, 0, 0, 0, 0, 0};
    }
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
  const int64_t kv_head_off = (int64_t)kvh * p.s_kh;
  const int64_t sc_head_off = (int64_t)kvh * p.s_sh;
  const int32_t* bt_row = p.bt + (int64_t)b * p.s_bt;

  for (int it = 0; it < CHUNKS / kAttnWaves; ++it) {
    const int t0 = split * kAttnSplitTokens + (it * kAttnWaves + w) * kAttnChunk;
    if (t0 >= kv_end) break;  // wave-uniform; later chunks of this wave are further out

    // ---- K tile: two 16-token sub-tiles, lane (tt, g) loads bytes [32g, 32g+32) of token tt.
    v8h kf[2][NU];
    float ksc[2][4], vsc[2][4];
    uint32_t vraw[4][4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ts = t0 + 16 * j;
      if (ts < kv_end) {
        const int page = bt_row[ts / p.PAGE];
        const int off0 = ts % p.PAGE;
        const int8_t* krow = p.kc + (int64_t)page * p.s_kp + (int64_t)(off0 + r) * p.s_ko + kv_head_off + DS * g;
        const v4i k0 = *reinterpret_cast<const v4i*>(krow);
        kf[j][0] = i8x8_to_h8((uint32_t)k0.x, (uint32_t)k0.y);
        kf[j][1] = i8x8_to_h8((uint32_t)k0.z, (uint32_t)k0.w);
        if constexpr (NU == 4) {
          const v4i k1 = *reinterpret_cast<const v4i*>(krow + 16);
          kf[j][2] = i8x8_to_h8((uint32_t)k1.x, (uint32_t)k1.y);
          kf[j][3] = i8x8_to_h8((uint32_t)k1.z, (uint32_t)k1.w);
        }
        const int64_t sbase = (int64_t)page * p.s_sp + sc_head_off;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t si = sbase + (int64_t)(off0 + 4 * g + i) * p.s_so;
          ksc[j][i] = load_scale<ST>(p.ks, si);
          vsc[j][i] = load_scale<ST>(p.vs, si);
        }
      } else {
#pragma unroll
        for (int u = 0; u < NU; ++u) kf[j][u] = v8h{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) { ksc[j][i] = 0.f; vsc[j][i] = 0.f; }
      }
    }
    // ---- V tile: lane (tq = lane/8, dq = lane%8) loads 4 tokens x (D/8) bytes.
    {
      const int tq = lane >> 3, dq = lane & 7;
      const int ts = t0 + 4 * tq;
      const int j = tq >> 2;  // sub-tile
      const bool ok = (t0 + 16 * j) < kv_end;
      const int page = ok ? bt_row[(t0 + 16 * j) / p.PAGE] : 0;
      const int off = (t0 + 16 * j) % p.PAGE + (ts - t0 - 16 * j);
      constexpr int DB = D / 8;  // bytes per lane per token: 16 (D=128) or 8 (D=64)
      const int8_t* vrow = p.vc + (int64_t)page * p.s_kp + (int64_t)off * p.s_ko + kv_head_off + DB * dq;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (DB == 16) {
          v4i v = ok ? *reinterpret_cast<const v4i*>(vrow + (int64_t)i * p.s_ko) : v4i{0, 0, 0, 0};
          vraw[i][0] = v.x; vraw[i][1] = v.y; vraw[i][2] = v.z; vraw[i][3] = v.w;
        } else {
          v2i v = ok ? *reinterpret_cast<const v2i*>(vrow + (int64_t)i * p.s_ko) : v2i{0, 0};
          vraw[i][0] = v.x; vraw[i][1] = v.y; vraw[i][2] = 0; vraw[i][3] = 0;
        }
      }
      // transpose and store: Vt[d][token] for d in [DB*dq, DB*dq + DB), tokens 4tq..4tq+3
#pragma unroll
      for (int c = 0; c < DB / 4; ++c) {
        uint32_t x[4] = {vraw[0][c], vraw[1][c], vraw[2][c], vraw[3][c]};
        uint32_t y[4];
        transpose4x4(x, y);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          *reinterpret_cast<uint32_t*>(vt + (DB * dq + 4 * c + e) * kAttnVtPitch + 4 * tq) = y[e];
      }
    }

    // ---- S^T = K . Q^T, online softmax, P^T operand.
    v8h pf[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float s[2][4];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        v4f c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < NU; ++u) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[j][u], qf[rb][u], c, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = t0 + 16 * j + 4 * g + i;
          s[j][i] = (t <= qpos[rb]) ? c[i] * (ksc[j][i] * p.scale_log2) : -INFINITY;
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
      m_run[rb] = m_new;
#pragma unroll
      for (int db = 0; db < ND; ++db) acc[rb][db] *= alpha;
    }

    // ---- O^T += V^T . P^T  (A-operand: lane (d, g) holds tokens {4g..4g+3, 16+4g..16+4g+3} of d)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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
        for (int db = 0; db < ND; ++db)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float* dst = &o_lds[rb * 16 + r][db * 16 + 4 * g + i];
            const float v = acc[rb][db][i] * wscale[rb];
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

  // ---- Cross-split merge: publish this split, the last to arrive combines in split order.
  const int64_t prog_base = (int64_t)prog * p.n_splits;
  float* opart = p.part;
  float* mlpart = p.part + (int64_t)gridDim.y * gridDim.z * p.n_splits * ROWS * D;
  for (int e = threadIdx.x; e < ROWS * D; e += blockDim.x) {
    const int row = e / D, d = e % D;
    publish(opart + ((prog_base + split) * ROWS + row) * D + d, o_lds[row][d]);
  }
  if (threadIdx.x < ROWS) {
    float* mlp = mlpart + ((prog_base + split) * ROWS + threadIdx.x) * 2;
    publish(mlp, ml_lds[0][0][threadIdx.x]);
    publish(mlp + 1, ml_lds[0][1][threadIdx.x]);
  }
  if (!arrive_last(p.counters + prog, n_active, &s_last)) return;
  for (int e = threadIdx.x; e < ROWS * DCH; e += blockDim.x) {
    const int row = e / DCH, d0 = (e % DCH) * 8;
    const int qi = qc * p.QPP + row / G;
    if (!(row < p.QPP * G && qi < q_len)) continue;
    const int head = kvh * G + row % G;
    float mx = -INFINITY;
    for (int s = 0; s < n_active; ++s) mx = fmaxf(mx, collect(mlpart + ((prog_base + s) * ROWS + row) * 2));
    const float ms = (mx == -INFINITY) ? 0.f : mx;
    float o[8];
    float l = 0.f;
    for (int s = 0; s < n_active; ++s) {
      const float* mlp = mlpart + ((prog_base + s) * ROWS + row) * 2;
      const float ws = fast_exp2(collect(mlp) - ms);
      const float ls = ws * collect(mlp + 1);
      l = (s == 0) ? ls : l + ls;
      const float* op = opart + ((prog_base + s) * ROWS + row) * D + d0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = ws * collect(op + i);
        o[i] = (s == 0) ? v : o[i] + v;
      }
    }
    const float inv = (l == 0.f) ? 0.f : 1.f / l;
    v8h out;
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = (_Float16)(o[i] * inv);
    *reinterpret_cast<v8h*>(p.out + (int64_t)b * p.s_ob + (int64_t)qi * p.s_ot + (int64_t)head * p.s_oh + d0) = out;
  }
}

}  // namespace specq
