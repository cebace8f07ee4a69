// INT8 paged-KV verification attention for gfx950.
//
// Computes, for every active sequence b, KV head h, query token i (of the q_len appended to
// the context) and query head of the GQA group, the reference's kernels.py:178-236:
//   s_t = (q . k_t) * ks_t * sm_scale   for t <= L - q_len + i   (causal on absolute position)
//   p_t = softmax_t(s)                  (online, rows with no visible key give 0)
//   o   = sum_t fp16(p_t * vs_t) * v_t  (the V scale is folded into P before the PV product)
// K/V are int8 [pages, PAGE, H_KV, D] reached through a block table; scales are fp16 or fp32.
// Tokens on a page whose block-table id lies outside [0, pages) are masked (read nothing,
// contribute nothing); the reference reads whatever address such an id names.
//
// MI355X schedule:
//  * One workgroup = (KV split, KV head, query chunk of QPP tokens, sequence).  The QPP * G
//    query rows sharing the KV head are packed into RB 16-row blocks, so a fused verification
//    program reads each K/V byte once for all (k+1) * G rows.
//  * Split length follows the work on the device: a split is a whole number of 128-token
//    units, as many as make (active sequences) x (KV heads) x (splits) reach the CU count for
//    a sequence filling the block table, at most 8192 tokens and at most 64 splits, and at
//    least 256 tokens (384 once the block table holds 4096 tokens or more), the units spread
//    evenly over the splits (attn_split_units).  It depends only on the block table's
//    capacity and the number of active sequences, so a QPP=1 and a fused program, and an eager and a plan-mode call, cut
//    a sequence at the same tokens, and the page ids of a split can be fetched before the
//    sequence's length is known.
//  * Eight waves (two per SIMD, so one wave's MFMA and LDS latencies hide behind the other's
//    arithmetic) take interleaved 16-token chunks of the split (chunk c, one page sub-tile,
//    goes to wave c % 8) and stream them through a wave-private LDS ring of 4 slots by LDS DMA
//    (global_load_lds_dwordx4, 64-bit per-lane addresses through the block table): three
//    chunks per wave (12 KB, 96 KB per CU) are in flight while one is multiplied, with no
//    register cost.  K and V rows land in LDS with their 16-byte granules XOR-swizzled by
//    token, so the MFMA-layout reads below are bank-conflict free.  Every iteration issues
//    the same DMAs (past the end they read a fixed valid address), so each s_waitcnt vmcnt is
//    a compile-time constant; the DMAs are inline asm the compiler does not track, so all
//    waits on them are the kernel's own, and each slot is its own LDS variable.  Page ids of
//    all of a wave's chunks are fetched with one load per lane at the start and picked out
//    with v_readlane.
//  * S^T = K . Q^T on v_mfma_f32_16x16x32_f16 with K (int8 -> fp16 in registers) as the A
//    operand: operand row x is token perm(x) of the chunk.  The result lands with the query
//    row in lane % 16, the B-operand layout of the PV product, so P never moves between
//    lanes.  perm interleaves the token rows so that the two 32-lane halves of each V read
//    below touch rows of opposite parity (different LDS bank halves).
//  * O^T = V^T . P^T on v_mfma_f32_16x16x16f16 with V^T as the A operand: lane (i, g) reads
//    bytes [ND*i, ND*i + ND) of its 4 tokens with 4 LDS reads and transposes them with v_perm
//    (4x4 byte transposes), so O^T block b row i is d = ND*i + b.  The O accumulator has the
//    query row in lane % 16, so the online-softmax rescale is lane local; the row max across
//    the four 16-lane rows uses the gfx950 row-swap permutes.
//  * The waves merge through LDS: wave v + 4 writes its rescaled O into the idle ring slots
//    of the pair (v, v + 4), wave v adds it to its own and writes the pair's sum back, then
//    all threads sum the four pairs in order.  Splits merge in
//    split order through the workspace (16-byte hand-offs, valid rows only, last workgroup to
//    arrive).  Split boundaries and the chunk-to-wave assignment are fixed token positions,
//    so a row's result is bit-identical whether it is computed by a QPP=1 or a fused program,
//    eagerly or from a plan-mode graph.
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
  int n_pages;         // pages in the K/V pool: block-table ids outside [0, n_pages) are masked
  const int32_t* ctx_len;
  _Float16* out; int64_t s_ob, s_ot, s_oh;
  const int32_t* plan;
  int B_grid, n_seqs, q_len, ql_grid;
  int G, QPP, n_qc, H_KV, PAGE;
  int n_splits;        // the most splits any active count of sequences gives (workspace stride)
  int target_wgs;      // workgroups the split length aims at (the device's CUs)
  float scale_log2;    // sm_scale * log2(e)
  float* part;         // [progs][n_splits][rows][D] unnormalised O, then [progs][n_splits][rows][2] (m, l)
  int32_t* counters;   // [progs]
  uint64_t* tl;        // diagnostics build only: per-workgroup timestamps (null otherwise)
  int tl_cap;          // workgroups tl has room for
};


constexpr int kAttnChunk = 16;                      // tokens per wave iteration (one page sub-tile)
constexpr int kAttnWaves = 8;                       // two per SIMD
constexpr int kAttnThreads = kAttnWaves * 64;
constexpr int kAttnUnit = kAttnChunk * kAttnWaves;  // 128 tokens: one chunk of every wave
constexpr int kAttnMinUnits = 2;                    // shortest split: 256 tokens (384 from 4096 tokens)
// Longest split: 8192 tokens, 64 chunks per wave, whose page ids the wave's 64 lanes hold.  At
// 32 sequences x 8 KV heads and 4096 tokens the programs alone fill the CUs: one split each runs
// one round of 256 workgroups, where 4096-token splits ran two rounds of 256 (91.6 us).
constexpr int kAttnMaxUnits = 64;
constexpr int kAttnMergeMax = 64;                   // most splits one program merges
constexpr int kAttnRing = 4;                        // LDS chunk slots per wave
// Largest unnormalised probability p = exp2(s - m) the lazy running max lets through (2^6):
// p * vs stays at most 64 * 65504 / 127 < 65504, inside fp16, for the V scale of any fp16 row
// quantised to int8 (vs <= 65504 / 127).
constexpr float kAttnLazyP = 64.f;
constexpr int64_t kAttnMaxTokens = (int64_t)kAttnUnit * kAttnMaxUnits * kAttnMergeMax;  // 524288

// 128-token units per split for a sequence of L tokens when `pairs` (sequence, KV head) pairs
// are active and the device has `target` CUs.
__host__ __device__ inline int attn_split_units(int L, int pairs, int target) {
  const int n = L > 0 ? (L + kAttnUnit - 1) / kAttnUnit : 1;
  const int pr = pairs > 0 ? pairs : 1;
  const int want = pr >= target ? 1 : (target + pr - 1) / pr;
  int u = (n + want - 1) / want;
  const int u_min = (n + kAttnMergeMax - 1) / kAttnMergeMax;
  if (u < u_min) u = u_min;
  // Splits of one or two chunks per wave leave the merge and hand-off to dominate; from 4096
  // tokens (32 units) up the shortest split is three units (B = 1, ctx 4096: 25.0 -> 22.9 us in
  // a graph), while shorter sequences keep two (B = 1, ctx 1024, k = 0: two units are faster).
  const int u_floor = n >= 32 ? kAttnMinUnits + 1 : kAttnMinUnits;
  if (u < u_floor) u = u_floor;
  if (u > kAttnMaxUnits) u = kAttnMaxUnits;
  // Even out the splits (a 33-unit sequence in 32-unit splits becomes 17 + 16, not 32 + 1).
  const int ns = (n + u - 1) / u;
  return (n + ns - 1) / ns;
}

// Operand row x of a 16-token sub-tile holds token attn_perm(x): rows 4g..4g+3 (one lane group
// of the S^T result) hold tokens 2e + (g & 1) + 8 (g >> 1), e = 0..3.
__device__ __forceinline__ int attn_perm(int x) { return 2 * (x & 3) + ((x >> 2) & 1) + 8 * (x >> 3); }

// Granule slot key of chunk token T (GR 16-byte granules per row): granule q of the row is
// stored in slot q ^ key(T).
template <int GR>
__device__ __forceinline__ int attn_key(int T) { return (T + (T >> 3)) & (GR - 1); }

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

// Max over the four 16-lane rows of a lane's column (lanes l, l^16, l^32, l^48), with the
// gfx950 row-swap permutes (no LDS round trip).
__device__ __forceinline__ float group_max4(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float m1 = fmaxf(__builtin_bit_cast(float, (uint32_t)a[0]), __builtin_bit_cast(float, (uint32_t)a[1]));
  const uint32_t v = __builtin_bit_cast(uint32_t, m1);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)b[0]), __builtin_bit_cast(float, (uint32_t)b[1]));
}

// Unsigned max over the four 16-lane rows of a lane's column (lanes l, l^16, l^32, l^48).
__device__ __forceinline__ uint32_t group_umax4(uint32_t u) {
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const uint32_t m1 = max((uint32_t)a[0], (uint32_t)a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(m1, m1, false, false);
  return max((uint32_t)b[0], (uint32_t)b[1]);
}

// LDS DMA (lds wave-uniform): lane l's 16 bytes land at lds + 16 l (dwordx4), its dword at
// lds + 4 l (dword), its 16-bit value in the low half of the dword at lds + 4 l (ushort).  The
// K/V DMAs are buffer loads: the chunk's page sub-tile is the resource base (scalar), the lane's
// granule offset within it the VGPR offset, which is the same for every chunk, so a chunk's
// addresses cost no vector arithmetic; an offset with bit 31 set is out of range and writes
// zeros.  The scale DMA reads from 64-bit per-lane addresses (lanes read K or V scales).
// Issued as inline asm: the compiler then neither counts these loads nor makes LDS accesses
// wait for them, and every dependence on them is an explicit wait_vmcnt of the kernel (its own
// loads only ever get stricter waits, which stays correct).  An LDS DMA reads M0 one wait state
// after it is written, hence the s_nop.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_ptr_t)p;
}
// Raw buffer resource over [base, base + 2^31): offsets with bit 31 set are out of range.
__device__ __forceinline__ v4i attn_rsrc(const void* base) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  return v4i{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xFFFFu), (int)kOOB, kRsrcWord3};
}
__device__ __forceinline__ void dma16_rs(v4i rs, uint32_t voff, uint8_t* lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rs),
               "s"(lds_addr(lds))
               : "memory", "m0");
}
__device__ __forceinline__ void dma4_global(const void* src, uint8_t* lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds_addr(lds)) : "memory", "m0");
}
__device__ __forceinline__ void dma2_global(const void* src, uint8_t* lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_ushort %0, off" ::"v"(src), "s"(lds_addr(lds)) : "memory", "m0");
}
// 64-bit value of lane `l` (wave-uniform l).
__device__ __forceinline__ int64_t readlane64(int64_t v, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), l);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// LDS bytes of one ring slot: K, V, then ks / vs (one dword per lane).
template <int D>
struct AttnSlot { static constexpr int value = 2 * kAttnChunk * D + 256; };

// The kernel body for RB 16-row query blocks, on LDS arrays sized for RBL >= RB blocks (the
// plan-mode launch below runs the body of the active rows' RB on arrays sized for the largest).
template <int D, int RB, typename ST, int RBL>
__device__ __forceinline__ void paged_attn_body(const AttnParams& p, uint8_t (&ring0)[kAttnWaves][AttnSlot<D>::value],
                                                uint8_t (&ring1)[kAttnWaves][AttnSlot<D>::value],
                                                uint8_t (&ring2)[kAttnWaves][AttnSlot<D>::value],
                                                uint8_t (&ring3)[kAttnWaves][AttnSlot<D>::value],
                                                float (&ml_lds)[kAttnWaves][2][RBL * 16],
                                                float (&row_lds)[2][RBL * 16],
                                                v8h (&q_lds)[RBL][D / 32][64], int& s_last) {
  static_assert(RB <= RBL, "LDS arrays hold the row blocks");
  constexpr int NU = D / 32;              // MFMA K-steps over the head dimension
  constexpr int ND = D / 16;              // 16-row d blocks of O^T = V bytes per lane per token
  constexpr int GR = D / 16;              // 16-byte granules per K/V row
  constexpr int KV4 = D / 64;             // 16-byte K granules per lane per token
  constexpr int DS = D / 4;               // head-dim bytes per lane per token (K) or row (Q)
  constexpr int ROWS = RB * 16;
  constexpr int NS = kAttnRing;
  constexpr int NT = kAttnThreads;
  constexpr int KB = kAttnChunk * D;      // K (or V) bytes per chunk
  constexpr int SC = 2 * KB;              // offset of the chunk's scale dwords in a slot
  constexpr int SLOT = AttnSlot<D>::value;
  static_assert(SLOT == 2 * KB + 256, "slot layout");
  constexpr int NDMA = KB / 1024;         // 1 KB DMA instructions for K, and again for V
  constexpr int NVM = 2 * NDMA + 1;       // DMA instructions per chunk (K, V, scales)
  constexpr int HALF = 8 * D * 4;         // bytes of 8 fp32 O rows: one half of a merge block
  static_assert(D == 64 || D == 128, "head dim");
  static_assert(RB >= 1 && RB <= NS && HALF <= SLOT, "merge block halves fit a ring slot");
  static_assert((NS - 1) * NVM <= 63, "vmcnt range");
  static_assert(NS == 4, "four ring variables");
  tl_mark(p.tl, p.tl_cap, 0);  // diagnostics build: workgroup start

  int n_seqs = p.n_seqs, q_len = p.q_len;
  if (p.plan != nullptr) {
    n_seqs = min(max(p.plan[0], 0), p.B_grid);
    q_len = min(max(p.plan[1], 0), p.ql_grid);
  }
  n_seqs = uniform(n_seqs);
  q_len = uniform(q_len);
  // Splits are sized from the block table's capacity (not the sequence's own length), so the
  // page ids of the split can be fetched together with the context length and Q: one memory
  // round trip before the first K/V DMA.
  const int cap = p.max_pages * p.PAGE;
  const int split_tokens = kAttnUnit * attn_split_units(cap, n_seqs * p.H_KV, p.target_wgs);
  // The grid is one-dimensional: workgroup id = program * splits + split (the exception for
  // eager calls with several query chunks and long splits is below), with the split count
  // of the active sequences, so the workgroups that have work are the first ones dispatched and
  // a plan-mode grid (sized for the worst active count) carries few idle workgroups.  (The
  // GEMMs' interleaved split order does not pay here: it puts each KV head's workgroups on one
  // XCD, and every XCD then fetches the 128-byte lines that hold the scales of all the heads --
  // 90.1 instead of 79.2 MB per launch at B = 8, k = 8, context 4096, for no time gained.)
  const int ns_act = (cap + split_tokens - 1) / split_tokens;
  int prog, split;
  if (p.n_qc == 1 || p.plan != nullptr || ns_act > 2) {
    prog = (int)blockIdx.x / ns_act;
    split = (int)blockIdx.x - prog * ns_act;
  } else {
    // Eager calls with several query chunks per KV head (QPP < q_len) and long splits (at most
    // two per sequence) place the n_qc programs that read one (sequence, KV head, split) range
    // 8 workgroups apart, in blocks of 8 ranges: they share blockIdx.x mod 8 -- one XCD -- and
    // run at the same time, so that XCD's L2 serves the range's K/V lines to all of them
    // instead of every XCD fetching them.  Measured with QPP = 1: B = 32, context 4096,
    // k = 1..8: 10-17 % faster; B = 16 and B = 32 at context 1024 and B = 16 at 4096: up to
    // 10 % faster (one point 1 % slower); with three or more splits per sequence the order
    // changed times by -4..+3 %, so those keep the program-major order.
    const int nr = n_seqs * p.H_KV * ns_act;  // (sequence, KV head, split) ranges
    const int id = (int)blockIdx.x, nq = p.n_qc;
    const int full = (nr / 8) * 8;
    int range, qc;
    if (id < full * nq) {
      const int blk = id / (8 * nq), rem = id - blk * (8 * nq);
      qc = rem / 8;
      range = blk * 8 + rem % 8;
    } else {
      const int rem = id - full * nq, tail = nr - full;
      if (tail <= 0 || rem >= tail * nq) return;
      qc = rem / tail;
      range = full + rem % tail;
    }
    split = range % ns_act;
    prog = (range / ns_act) * nq + qc;
  }
  if (prog >= n_seqs * p.H_KV * p.n_qc) return;
  const int qc = prog % p.n_qc, kvh = (prog / p.n_qc) % p.H_KV, b = prog / (p.n_qc * p.H_KV);
  if (qc * p.QPP >= q_len) return;
  const int s0 = split * split_tokens;
  const int L_raw = p.ctx_len[b];

  const int lane = lane_id(), w = uniform(wave_id()), g = lane >> 4, r = lane & 15;
  const int G = p.G;
  auto ring_of = [&](auto ic, int wave) -> uint8_t* {
    constexpr int i = decltype(ic)::value;
    if constexpr (i == 0) return ring0[wave];
    else if constexpr (i == 1) return ring1[wave];
    else if constexpr (i == 2) return ring2[wave];
    else return ring3[wave];
  };

  float m_run[RB], l_run[RB];
  v4f acc[RB][ND];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m_run[rb] = -INFINITY;
    l_run[rb] = 0.f;
#pragma unroll
    for (int db = 0; db < ND; ++db) acc[rb][db] = v4f{0.f, 0.f, 0.f, 0.f};
  }

  // This wave's chunks of the split: chunk `it` is the 16 tokens from s0 + 16 (w + 8 it), one
  // page sub-tile.
  auto chunk_t0 = [&](int it) { return s0 + kAttnChunk * (w + kAttnWaves * it); };
  const int32_t* bt_row = p.bt + (int64_t)b * p.s_bt;
  // Page of the wave's chunk `lane` within the split and the block table (at most 64 chunks);
  // chunks at or past kv_end never use theirs.
  int page_v;
  {
    const int ts = chunk_t0(lane);
    page_v = (ts < s0 + split_tokens && ts < cap) ? bt_row[ts / p.PAGE] : 0;
  }
  // Q fragments: thread t stages fragments t, t + NT, ... of [rb][u][lane].
  constexpr int QF = (RB * NU * 64 + NT - 1) / NT;
  v8h qtmp[QF];
#pragma unroll
  for (int i = 0; i < QF; ++i) {
    const int f = threadIdx.x + NT * i;
    const int rb = f / (NU * 64), u = (f / 64) % NU, ln = f % 64;
    const int row = rb * 16 + (ln & 15);
    const int qi = qc * p.QPP + row / G;
    const bool ok = f < RB * NU * 64 && row < p.QPP * G && qi < q_len;
    const int head = kvh * G + row % G;
    const _Float16* src = ok ? p.q + (int64_t)b * p.s_qb + (int64_t)qi * p.s_qt + (int64_t)head * p.s_qh + DS * (ln >> 4) + 8 * u
                             : p.q;
    const v8h x = *reinterpret_cast<const v8h*>(src);
    qtmp[i] = ok ? x : v8h{0, 0, 0, 0, 0, 0, 0, 0};
  }

  // The context length (a scalar load, in flight with the page ids and Q).
  const int L = uniform(min(L_raw, cap));
  const int kv_end = L - q_len + min(qc * p.QPP + p.QPP, q_len);
  // Split 0 always runs, so rows with no visible key still get their zero output.
  if (split > 0 && s0 >= kv_end) return;
  const int n_active = kv_end > split_tokens ? (kv_end + split_tokens - 1) / split_tokens : 1;
  const int s1 = min(s0 + split_tokens, kv_end);
  const int n_it = uniform(s1 > s0 + kAttnChunk * w ? (s1 - s0 - kAttnChunk * w + kAttnUnit - 1) / kAttnUnit : 0);
  int qpos[RB];  // absolute position of the query row this lane holds in each row block
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = rb * 16 + r;
    const int qi = qc * p.QPP + row / G;
    const bool valid = (row < p.QPP * G) && (qi < q_len);
    qpos[rb] = valid ? (L - q_len + qi) : -1;
  }

  // Page ids and Q fragments arrive together (one memory round trip); Q goes to LDS before any
  // DMA is issued, so no LDS store ever waits behind the ring's DMA.
  wait_vmcnt<0>();
  tl_mark(p.tl, p.tl_cap, 1);  // diagnostics build: page ids, Q and the length have landed
#pragma unroll
  for (int i = 0; i < QF; ++i) {
    const int f = threadIdx.x + NT * i;
    if (f < RB * NU * 64) (&q_lds[0][0][0])[f] = qtmp[i];
  }

  // Chunk-invariant per-lane parts of the DMA addresses: the byte offset of the lane's K/V
  // granule within the chunk's page sub-tile (DMA i covers chunk tokens 64 i / GR ..; below
  // 2^31, which the host checks), and the address of its scale within the chunk's first token.
  // Lanes l < 16 fetch ks of token perm(l), 16 <= l < 32 vs of token perm(l - 16), lanes 32..
  // repeat lanes 0..31.
  uint32_t kvoff[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int gi = 64 * i + lane, T = gi / GR, s = gi % GR;
    kvoff[i] = (uint32_t)((int64_t)T * p.s_ko + 16 * (s ^ attn_key<GR>(T)));
  }
  const int sc_T = attn_perm(lane & 15);
  const uint8_t* sc_src = reinterpret_cast<const uint8_t*>((lane & 16) ? p.vs : p.ks);
  const uint8_t* sc_lane = sc_src + (int64_t)sc_T * p.s_so * (int64_t)sizeof(ST);
  // Per-chunk bases, lane c holding the wave's chunk c: the byte offset of the chunk's page
  // sub-tile of this KV head in the K/V cache, and that of its first token's scales.  Chunks
  // at or past the wave's last use page 0 (their DMAs read nothing or a fixed valid address).
  // Chunks whose page id lies outside the pool read nothing and are masked like tokens past
  // kv_end (bit c of bad_chunks: the wave's chunk c).
  const bool page_ok = (uint32_t)page_v < (uint32_t)p.n_pages;
  const uint64_t bad_chunks = __builtin_amdgcn_ballot_w64(lane < n_it && !page_ok);
  int64_t kv_base_v, sc_base_v;
  {
    const int pg = lane < n_it && page_ok ? page_v : 0;
    const int tk = chunk_t0(lane) % p.PAGE;
    kv_base_v = (int64_t)pg * p.s_kp + (int64_t)tk * p.s_ko + (int64_t)kvh * p.s_kh;
    sc_base_v = ((int64_t)pg * p.s_sp + (int64_t)tk * p.s_so + (int64_t)kvh * p.s_sh) * (int64_t)sizeof(ST);
  }
  // Issue the DMAs of chunk `it` into ring slot SL.  K/V granules of chunks past the wave's
  // last or on a page outside the pool, and of tokens at or past kv_end, are out of range
  // (zeros); their scales read a fixed valid address.
  auto issue = [&](auto slc, int it) __attribute__((always_inline)) {
    uint8_t* dst = ring_of(slc, w);
    const int li = min(it, 63);
    const bool real = it < n_it && ((bad_chunks >> li) & 1) == 0;
    const int t0 = chunk_t0(it);
    const int64_t kb = readlane64(kv_base_v, li);
    const int64_t sb = readlane64(sc_base_v, li);
    const v4i rk = attn_rsrc(p.kc + kb), rv = attn_rsrc(p.vc + kb);
    if (real && t0 + kAttnChunk <= kv_end) {
#pragma unroll
      for (int i = 0; i < NDMA; ++i) dma16_rs(rk, kvoff[i], dst + 1024 * i);
#pragma unroll
      for (int i = 0; i < NDMA; ++i) dma16_rs(rv, kvoff[i], dst + KB + 1024 * i);
      const uint8_t* src = sc_lane + sb;
      if constexpr (sizeof(ST) == 4) dma4_global(src, dst + SC);
      else dma2_global(src, dst + SC);
    } else {
#pragma unroll
      for (int i = 0; i < NDMA; ++i) {
        const bool ok = real && t0 + (64 * i + lane) / GR < kv_end;
        dma16_rs(rk, oob_unless(ok, kvoff[i]), dst + 1024 * i);
      }
#pragma unroll
      for (int i = 0; i < NDMA; ++i) {
        const bool ok = real && t0 + (64 * i + lane) / GR < kv_end;
        dma16_rs(rv, oob_unless(ok, kvoff[i]), dst + KB + 1024 * i);
      }
      const bool ok = real && t0 + sc_T < kv_end;
      const uint8_t* src = ok ? sc_lane + sb : sc_src;
      if constexpr (sizeof(ST) == 4) dma4_global(src, dst + SC);
      else dma2_global(src, dst + SC);
    }
  };

  // Up to two row blocks the Q fragments stay in registers for the whole loop (RB * NU * 4
  // VGPRs); deeper packings read them from LDS per chunk.
  constexpr bool QREG = RB <= 2;
  v8h qreg[QREG ? RB : 1][NU];
  auto qfrag = [&](int rb, int u) -> v8h {
    if constexpr (QREG) return qreg[rb][u];
    else return q_lds[rb][u][lane];
  };
  // One chunk in two stages.  Stage A reads the chunk's K, V and scales from its ring slot,
  // converts K to fp16 and computes S^T = K . Q^T; stage B applies the scales and the causal
  // mask, runs the online softmax and accumulates O^T += V^T . P^T.  A wave issues stage A of
  // chunk it + 1 before stage B of chunk it, so the S^T MFMAs of one chunk are in flight
  // while the other's softmax runs.  Each chunk's arithmetic is unchanged, so the results do
  // not depend on the pipelining.
  struct Staged {
    v4f cs[RB];                // S^T of the chunk before the scales
    float ksc[4], vsc[4];      // K scale * sm_scale * log2(e), V scale, in operand order
    uint32_t vx[4][ND / 4];    // V bytes of operand slots 4g..4g+3
  };
  auto stage_a = [&](auto slc, Staged& st) __attribute__((always_inline)) {
    const uint8_t* kb = ring_of(slc, w);
    const uint8_t* vb = kb + KB;
    // K operands: lane (r, g) holds head-dim bytes [DS*g, DS*g + DS) of token perm(r).
    v8h kf[NU];
    {
      const int T = attn_perm(r), key = attn_key<GR>(T);
#pragma unroll
      for (int h = 0; h < KV4; ++h) {
        const v4i x = *reinterpret_cast<const v4i*>(kb + T * D + 16 * ((g * KV4 + h) ^ key));
        kf[2 * h] = i8x8_to_h8((uint32_t)x.x, (uint32_t)x.y);
        kf[2 * h + 1] = i8x8_to_h8((uint32_t)x.z, (uint32_t)x.w);
      }
    }
    // V^T operands: lane (r, g) reads bytes [ND*r, ND*r + ND) of tokens perm(4g + e), operand
    // slot 4g + e of the 16x16x16 product.
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int T = attn_perm(4 * g + e);
      const uint8_t* src = vb + T * D + 16 * (((ND * r) >> 4) ^ attn_key<GR>(T)) + ((ND * r) & 15);
      if constexpr (ND == 8) {
        const v2i x = *reinterpret_cast<const v2i*>(src);
        st.vx[e][0] = (uint32_t)x.x;
        st.vx[e][1] = (uint32_t)x.y;
      } else {
        st.vx[e][0] = *reinterpret_cast<const uint32_t*>(src);
      }
    }
    // Scales in operand order: dword 4g + e holds ks of token perm(4g + e), dword 16 + 4g + e
    // its vs (an fp16 scale in the low half).
    {
      const v4i kr = *reinterpret_cast<const v4i*>(kb + SC + 16 * g);
      const v4i vr = *reinterpret_cast<const v4i*>(kb + SC + 64 + 16 * g);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // Vector elements are copied out before the bit casts (a bit cast of a vector-element
        // expression reads the vector's first element).
        const int ki = kr[e], vi = vr[e];
        float kv, vv;
        if constexpr (sizeof(ST) == 4) {
          kv = __builtin_bit_cast(float, ki);
          vv = __builtin_bit_cast(float, vi);
        } else {
          kv = (float)__builtin_bit_cast(_Float16, (uint16_t)(ki & 0xFFFF));
          vv = (float)__builtin_bit_cast(_Float16, (uint16_t)(vi & 0xFFFF));
        }
        st.ksc[e] = kv * p.scale_log2;
        st.vsc[e] = vv;
      }
    }
    // S^T of every row block (RB independent MFMA chains).
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      v4f c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < NU; ++u) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[u], qfrag(rb, u), c, 0, 0, 0);
      st.cs[rb] = c;
    }
  };
  auto stage_b = [&](int it, const Staged& st) __attribute__((always_inline)) {
    const int t0 = chunk_t0(it);
    // A chunk on a page outside the pool: every token masked (wave-uniform).
    const bool bad = ((bad_chunks >> (it & 63)) & 1) != 0;
    // Zero V scale for tokens at or past kv_end and of masked chunks (their scale slots hold
    // the dummy address's).
    float vsc[4] = {st.vsc[0], st.vsc[1], st.vsc[2], st.vsc[3]};
    if (bad || t0 + kAttnChunk > kv_end) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (bad || t0 + attn_perm(4 * g + e) >= kv_end) vsc[e] = 0.f;
    }
    // Every row of the program sees every token of the chunk: no causal mask needed.
    const bool full = !bad && t0 + kAttnChunk - 1 <= L - q_len + qc * p.QPP;
    // Unnormalised probabilities against the row's running max m: p = exp2(s_raw * ksc - m)
    // (one fma; masked tokens 0).  While m = -inf every visible p is +inf.  The row max of p is
    // taken on the bit patterns (p >= 0, so their integer order is the numeric order).
    float pr[RB][4];
    uint32_t pbig = 0;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
      for (int e = 0; e < 4; ++e) pr[rb][e] = fast_exp2(fmaf(st.cs[rb][e], st.ksc[e], -m_run[rb]));
      if (!full) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (bad || t0 + attn_perm(4 * g + e) > qpos[rb]) pr[rb][e] = 0.f;
      }
      const uint32_t b0 = __builtin_bit_cast(uint32_t, pr[rb][0]), b1 = __builtin_bit_cast(uint32_t, pr[rb][1]);
      const uint32_t b2 = __builtin_bit_cast(uint32_t, pr[rb][2]), b3 = __builtin_bit_cast(uint32_t, pr[rb][3]);
      pbig = max(pbig, max(max(b0, b1), max(b2, b3)));
    }
    // Lazy running max: a row's m moves only when one of its p exceeds kAttnLazyP, i.e. a
    // score exceeds m by more than 6; m then becomes the row's exact max score and the
    // row's p, l and O are rescaled.  After a row's first chunk that is rare, so one wave-wide
    // test guards it.  The decision is the row's own (its four lanes see the same row max of p),
    // so each row's result does not depend on the rows packed with it.
    float alpha[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) alpha[rb] = 1.f;
    if (__builtin_amdgcn_ballot_w64(pbig > __builtin_bit_cast(uint32_t, kAttnLazyP)) != 0) {
      bool grew = false;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const uint32_t b0 = __builtin_bit_cast(uint32_t, pr[rb][0]), b1 = __builtin_bit_cast(uint32_t, pr[rb][1]);
        const uint32_t b2 = __builtin_bit_cast(uint32_t, pr[rb][2]), b3 = __builtin_bit_cast(uint32_t, pr[rb][3]);
        const uint32_t rowp = group_umax4(max(max(b0, b1), max(b2, b3)));
        float s[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s[e] = st.cs[rb][e] * st.ksc[e];
          if (!full && (bad || t0 + attn_perm(4 * g + e) > qpos[rb])) s[e] = -INFINITY;
        }
        const float rmax = group_max4(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
        if (rowp > __builtin_bit_cast(uint32_t, kAttnLazyP)) {
          alpha[rb] = fast_exp2(m_run[rb] - rmax);  // 0 from m = -inf
          m_run[rb] = rmax;
          grew = true;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            pr[rb][e] = s[e] == -INFINITY ? 0.f : fast_exp2(fmaf(st.cs[rb][e], st.ksc[e], -rmax));
        }
      }
      // alpha is exactly 1 for every row whose m did not move.
      if (__builtin_amdgcn_ballot_w64(grew) != 0) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int db = 0; db < ND; ++db) acc[rb][db] *= alpha[rb];
      }
    }
    v4h pf[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      l_run[rb] = l_run[rb] * alpha[rb] + ((pr[rb][0] + pr[rb][1]) + (pr[rb][2] + pr[rb][3]));
#pragma unroll
      for (int e = 0; e < 4; ++e) pf[rb][e] = (_Float16)f32_opaque(pr[rb][e] * vsc[e]);  // fp32 product, then fp16 (kernels.py:232)
    }
    // V bytes to d-major: vt[db] = the 4 token bytes (operand slots 4g..4g+3) of d = ND*r + db.
#pragma unroll
    for (int c = 0; c < ND / 4; ++c) {
      const uint32_t x[4] = {st.vx[0][c], st.vx[1][c], st.vx[2][c], st.vx[3][c]};
      uint32_t y[4];
      transpose4x4(x, y);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v2h lo, hi;
        i8x4_to_h2x2(y[e], lo, hi);
        const v4h vf = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc[rb][4 * c + e] = __builtin_amdgcn_mfma_f32_16x16x16f16(vf, pf[rb], acc[rb][4 * c + e], 0, 0, 0);
      }
    }
  };

  // Chunk c lives in slot (c + 1) % NS, so the loop body fills slots 0, 1, 2, 3 in order, the
  // order in which the prologue first touches them.
  // Prologue: chunks 0 .. NS-2; the barrier makes every wave's Q fragments visible.
  static_for<0, NS - 1>([&](auto ic) __attribute__((always_inline)) {
    constexpr int i = decltype(ic)::value;
    issue(std::integral_constant<int, (i + 1) % NS>{}, i);
  });
  wg_barrier_lds();
  if constexpr (QREG) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int u = 0; u < NU; ++u) qreg[rb][u] = q_lds[rb][u][lane];
  }
  // Steady state, step it: issue chunk it + NS - 1 into the slot chunk it - 1 left (both its
  // stages have run), wait for chunk it + 1 (NS - 2 chunks may stay in flight), run stage A of
  // chunk it + 1, then stage B of chunk it.  Chunk it's staged state lives in st[it % 2]; NS is
  // even, so the index is a compile-time constant in the unrolled body.
  // The 64-row program at D = 128 has no registers for a second staged state and runs the two
  // stages of a chunk back to back (waiting for chunk it itself, NS - 1 chunks in flight).
  constexpr bool PIPE = !(RB == 4 && D == 128);
  static_assert(NS % 2 == 0, "staged state ping-pong");
  if constexpr (PIPE) {
    Staged st[2];
    wait_vmcnt<(NS - 2) * NVM>();  // chunk 0 has landed
    tl_mark(p.tl, p.tl_cap, 2);    // diagnostics build: first chunk landed
    if (n_it > 0) stage_a(std::integral_constant<int, 1 % NS>{}, st[0]);
    for (int base = 0; base < n_it; base += NS) {
      static_for<0, NS>([&](auto ic) __attribute__((always_inline)) {
        constexpr int i = decltype(ic)::value;
        const int it = base + i;
        issue(ic, it + NS - 1);
        wait_vmcnt<(NS - 2) * NVM>();
        if (it + 1 < n_it) stage_a(std::integral_constant<int, (i + 2) % NS>{}, st[(i + 1) & 1]);
        if (it < n_it) stage_b(it, st[i & 1]);
      });
    }
  } else {
    for (int base = 0; base < n_it; base += NS) {
      static_for<0, NS>([&](auto ic) __attribute__((always_inline)) {
        constexpr int i = decltype(ic)::value;
        const int it = base + i;
        issue(ic, it + NS - 1);
        wait_vmcnt<(NS - 1) * NVM>();
        if (it < n_it) {
          Staged st;
          stage_a(std::integral_constant<int, (i + 1) % NS>{}, st);
          stage_b(it, st);
        }
      });
    }
  }
  // Every DMA has landed before the ring is reused for the merge.
  wait_vmcnt<0>();
  tl_mark(p.tl, p.tl_cap, 3);       // diagnostics build: chunk loop done (wave 0)
  tl_mark_wave(p.tl, p.tl_cap, 8);  // ... and per wave (marks 8..15)

  // ---- Merge the eight waves.  Row statistics first; every wave's O is scaled to the
  // workgroup's row max.  Wave pair (v, v + 4) shares a merge region: row block rb in ring
  // slot rb, rows 0-7 in wave v's slot and rows 8-15 in wave v + 4's, granule c of row n at
  // c ^ n.  Wave v + 4 writes its O, wave v adds it to its own and writes the pair's sum, then
  // all threads add the four pair sums in pair order.
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
  tl_mark(p.tl, p.tl_cap, 7);  // diagnostics build: every wave's chunk loop done
  constexpr int QPR = D / 4;  // 4-float granules per row
  // Each row's workgroup statistics, once: the row max over the waves and, in wave 0, the sum
  // l = sum_w exp2(m_w - max) l_w in wave order, kept in LDS for the stores and the split
  // hand-off below (visible after the merge's next barrier).
  float wsc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = rb * 16 + r;
    float mv[kAttnWaves];
#pragma unroll
    for (int ww = 0; ww < kAttnWaves; ++ww) mv[ww] = ml_lds[ww][0][row];
    float mx = mv[0];
#pragma unroll
    for (int ww = 1; ww < kAttnWaves; ++ww) mx = fmaxf(mx, mv[ww]);
    const float ms = (mx == -INFINITY) ? 0.f : mx;
    wsc[rb] = fast_exp2(m_run[rb] - ms);
    if (w == 0 && g == 0) {
      float l = 0.f;
#pragma unroll
      for (int ww = 0; ww < kAttnWaves; ++ww) l += fast_exp2(mv[ww] - ms) * ml_lds[ww][1][row];
      row_lds[0][row] = mx;
      row_lds[1][row] = l;
    }
  }
  const int pr = w & 3;  // the wave pair
  // O^T rows 4g + e of block db hold d = ND (4g + e) + db: granule (ND / 4)(4g + e) + cc.
  auto merge_io = [&](auto rbc, bool store) __attribute__((always_inline)) {
    constexpr int rb = decltype(rbc)::value;
    float* half0 = reinterpret_cast<float*>(ring_of(rbc, pr));
    float* half1 = reinterpret_cast<float*>(ring_of(rbc, pr + 4));
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int cc = 0; cc < ND / 4; ++cc) {
        const int gran = (ND / 4) * (4 * g + e) + cc;
        float* dst = (r < 8 ? half0 : half1) + (r & 7) * D + 4 * (gran ^ r);
        v4f* a = &acc[rb][0];
        if (store) {
          *reinterpret_cast<v4f*>(dst) = v4f{a[4 * cc][e], a[4 * cc + 1][e], a[4 * cc + 2][e], a[4 * cc + 3][e]};
        } else {
          const v4f v = *reinterpret_cast<const v4f*>(dst);
#pragma unroll
          for (int k = 0; k < 4; ++k) a[4 * cc + k][e] += v[k];
        }
      }
  };
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int db = 0; db < ND; ++db) acc[rb][db] *= wsc[rb];
  if (w >= 4) static_for<0, RB>([&](auto rbc) __attribute__((always_inline)) { merge_io(rbc, true); });
  __syncthreads();
  if (w < 4) static_for<0, RB>([&](auto rbc) __attribute__((always_inline)) { merge_io(rbc, false); });
  __syncthreads();
  if (w < 4) static_for<0, RB>([&](auto rbc) __attribute__((always_inline)) { merge_io(rbc, true); });
  __syncthreads();
  auto pair_o = [&](int pp, int row, int c) -> v4f {
    const int n = row & 15, rb = row >> 4;
    const int wv = pp + ((n >> 3) << 2);
    const uint8_t* base = rb == 0 ? ring0[wv] : rb == 1 ? ring1[wv] : rb == 2 ? ring2[wv] : ring3[wv];
    return *reinterpret_cast<const v4f*>(reinterpret_cast<const float*>(base) + (n & 7) * D + 4 * (c ^ n));
  };
  auto row_stats = [&](int row, float& mx, float& l) {
    mx = row_lds[0][row];
    l = row_lds[1][row];
  };
  constexpr int ITEMS = (ROWS * QPR + NT - 1) / NT;
  v4f o[ITEMS];
  bool ivalid[ITEMS];
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int e = threadIdx.x + NT * it;
    const int row = e / QPR, c = e % QPR;
    const int qi = qc * p.QPP + row / G;
    ivalid[it] = e < ROWS * QPR && row < p.QPP * G && qi < q_len;
    o[it] = v4f{0.f, 0.f, 0.f, 0.f};
    if (ivalid[it]) {
      o[it] = pair_o(0, row, c);
#pragma unroll
      for (int pp = 1; pp < 4; ++pp) o[it] += pair_o(pp, row, c);
    }
  }
  typedef _Float16 v4h_t __attribute__((ext_vector_type(4)));
  // Each value is rounded to fp32 before the fp16 cast (f32_opaque keeps the compiler from
  // fusing a last multiply and the cast into one v_fma_mixlo with a single rounding, which it
  // does in some instantiations and not others, so programs of different row counts would
  // round a midpoint differently).
  auto store_row4 = [&](int e, v4f v) {
    const int row = e / QPR, d0 = (e % QPR) * 4;
    const int qi = qc * p.QPP + row / G;
    const int head = kvh * G + row % G;
    *reinterpret_cast<v4h_t*>(p.out + (int64_t)b * p.s_ob + (int64_t)qi * p.s_ot + (int64_t)head * p.s_oh + d0) =
        v4h_t{(_Float16)f32_opaque(v.x), (_Float16)f32_opaque(v.y), (_Float16)f32_opaque(v.z),
              (_Float16)f32_opaque(v.w)};
  };

  tl_mark(p.tl, p.tl_cap, 4);  // diagnostics build: waves merged
  if (n_active == 1) {
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      if (!ivalid[it]) continue;
      const int e = threadIdx.x + NT * it;
      float mx, l;
      row_stats(e / QPR, mx, l);
      const float inv = (l == 0.f) ? 0.f : 1.f / l;
      store_row4(e, o[it] * inv);
    }
    tl_mark_drained(p.tl, p.tl_cap, 6);  // diagnostics build: output stored
    return;
  }

  // ---- Cross-split merge: publish this split's valid rows (16 bytes per lane), the last to
  // arrive combines the splits in split order.
  const int64_t prog_base = (int64_t)prog * p.n_splits;
  const int64_t n_o = (int64_t)p.B_grid * p.H_KV * p.n_qc * p.n_splits * ROWS * D;  // floats of the O region
  const rsrc_t ors = make_rsrc(p.part + prog_base * ROWS * D, (uint32_t)(p.n_splits * ROWS * D * 4));
  float* mlpart = p.part + n_o;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
    if (ivalid[it]) {
      const int e = threadIdx.x + NT * it;
      publish16(ors, (uint32_t)((split * ROWS * QPR + e) * 16), __builtin_bit_cast(v4i, o[it]));
    }
  if (threadIdx.x < ROWS) {
    float mx, l;
    row_stats(threadIdx.x, mx, l);
    float* mlp = mlpart + ((prog_base + split) * ROWS + threadIdx.x) * 2;
    publish(mlp, mx);
    publish(mlp + 1, l);
  }
  tl_mark(p.tl, p.tl_cap, 5);  // diagnostics build: partials issued
  if (!arrive_last(p.counters + prog, n_active, &s_last, p.tl, p.tl_cap)) {
    tl_mark(p.tl, p.tl_cap, 6);  // diagnostics build: hand-off done (not the last split)
    return;
  }
  // Row weights of the splits, exp2(m_s - max) / l (l summed in split order), in LDS (the first
  // ring, no longer read).  Up to 16 splits the (m, l) pairs are loaded once, all in flight
  // together; more splits take a second pass.
  float* wts = reinterpret_cast<float*>(&ring0[0][0]);  // [ROWS][kAttnMergeMax]
  static_assert(kAttnWaves * SLOT >= 64 * kAttnMergeMax * 4, "split weights fit the first ring");
  constexpr int kMergeBatch = 16;
  if (threadIdx.x < ROWS) {
    const int row = threadIdx.x;
    float* wt = wts + row * kAttnMergeMax;
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
  // O rows: sum over splits in split order of weight * partial O.  All of a thread's items'
  // loads of SB splits are in flight together.
  constexpr int SB = ITEMS <= 2 ? 8 : (ITEMS <= 4 ? 4 : 2);  // at most 16 16-byte loads in flight per thread
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) o[it] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int s0m = 0; s0m < n_active; s0m += SB) {
    v4i t[SB][ITEMS];
#pragma unroll
    for (int u = 0; u < SB; ++u)
#pragma unroll
      for (int it = 0; it < ITEMS; ++it) {
        const int e = threadIdx.x + NT * it;
        t[u][it] = collect16(ors, oob_unless(ivalid[it] && s0m + u < n_active,
                                             (uint32_t)(((s0m + u) * ROWS * QPR + e) * 16)));
      }
#pragma unroll
    for (int u = 0; u < SB; ++u)
#pragma unroll
      for (int it = 0; it < ITEMS; ++it)
        if (ivalid[it] && s0m + u < n_active) {
          const int e = threadIdx.x + NT * it;
          o[it] += wts[(e / QPR) * kAttnMergeMax + s0m + u] * __builtin_bit_cast(v4f, t[u][it]);
        }
  }
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
    if (ivalid[it]) store_row4(threadIdx.x + NT * it, o[it]);
  tl_mark_drained(p.tl, p.tl_cap, 6);  // diagnostics build: splits merged and stored
}

// The ring slots are separate LDS variables (see the schedule notes); Q fragments are staged
// in MFMA B-operand order [rb][u][lane] of 16 bytes (zero for padding rows).
#define SPECQ_ATTN_LDS(RBL)                                                          \
  __shared__ __attribute__((aligned(16))) uint8_t ring0[kAttnWaves][AttnSlot<D>::value]; \
  __shared__ __attribute__((aligned(16))) uint8_t ring1[kAttnWaves][AttnSlot<D>::value]; \
  __shared__ __attribute__((aligned(16))) uint8_t ring2[kAttnWaves][AttnSlot<D>::value]; \
  __shared__ __attribute__((aligned(16))) uint8_t ring3[kAttnWaves][AttnSlot<D>::value]; \
  __shared__ float ml_lds[kAttnWaves][2][(RBL) * 16];                                 \
  __shared__ float row_lds[2][(RBL) * 16];                                            \
  __shared__ __attribute__((aligned(16))) v8h q_lds[RBL][D / 32][64];                 \
  __shared__ int s_last

template <int D, int RB, typename ST>
__global__ __launch_bounds__(kAttnThreads) void paged_attn_kernel(AttnParams p) {
  SPECQ_ATTN_LDS(RB);
  paged_attn_body<D, RB, ST, RB>(p, ring0, ring1, ring2, ring3, ml_lds, row_lds, q_lds, s_last);
}

// Plan-mode launch captured for programs of up to RBMAX row blocks: the active q_len (plan[1])
// fixes how many rows a program holds, and the body of that many row blocks runs (a row's
// result does not depend on the rows packed with it, so every choice is bit-identical).
template <int D, int RBMAX, typename ST>
__global__ __launch_bounds__(kAttnThreads) void paged_attn_plan_kernel(AttnParams p) {
  SPECQ_ATTN_LDS(RBMAX);
  const int q_len = min(max(p.plan[1], 0), p.ql_grid);
  const int rb = uniform(min(max((min(q_len, p.QPP) * p.G + 15) / 16, 1), RBMAX));
  if (rb == 1) {
    paged_attn_body<D, 1, ST, RBMAX>(p, ring0, ring1, ring2, ring3, ml_lds, row_lds, q_lds, s_last);
  } else if (rb == 2) {
    if constexpr (RBMAX >= 2) paged_attn_body<D, 2, ST, RBMAX>(p, ring0, ring1, ring2, ring3, ml_lds, row_lds, q_lds, s_last);
  } else if (rb == 3) {
    if constexpr (RBMAX >= 3) paged_attn_body<D, 3, ST, RBMAX>(p, ring0, ring1, ring2, ring3, ml_lds, row_lds, q_lds, s_last);
  } else {
    if constexpr (RBMAX >= 4) paged_attn_body<D, 4, ST, RBMAX>(p, ring0, ring1, ring2, ring3, ml_lds, row_lds, q_lds, s_last);
  }
}
#undef SPECQ_ATTN_LDS

}  // namespace specq
