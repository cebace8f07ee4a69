// W8A8 GEMM, weight-streaming schedule with LDS-shared activations (aligned fast path).
//
// Same arithmetic as w8a8_kernel (reference kernels.py:27-55): INT8 x INT8 products summed
// exactly in INT32, then (acc * sa[m]) * sw[n] in fp32 and one RNE cast to fp16.
//
// Built from measurements of how MI355X feeds a skinny GEMM:
//  * Weights are the MFMA A operand and stream from HBM straight into a register ring that
//    runs D K-steps (64 bytes of K each) ahead of the MFMAs.  The fastest source is the
//    packed layout (WL 1): 1 KB MFMA fragments stored K-step-major, fragment (t, s) of
//    16-row tile t and step s at (s * ntiles + t) KB, so the workgroups running at one time
//    sweep one compact window of memory front to back and every load is 1 KB contiguous.
//    The row-major weight (WL 0) is read as MFMA fragments directly (16 rows x 64 B per
//    instruction); each workgroup then starts its K walk at a staggered chunk so the
//    workgroups do not all hit the same column range of the rows at once.
//  * Activations (small, L2 resident) are the B operand.  Reading them from L2 into every
//    wave's registers costs more than the weight stream itself once M > 16, so a workgroup
//    stages them once in LDS: chunks of KC bytes of K for all its token rows in a ring of
//    NSLOT slots, filled NSLOT-1 chunks ahead by LDS DMA (buffer_load ... lds) with 4 rows x
//    256 contiguous bytes per instruction.  The DMA lanes fetch 16-byte pieces in an XOR-swizzled order (piece c of
//    row r lands in slot c ^ (r % 16)), so the MFMA-layout ds_read_b128s that consume them
//    are bank-conflict free.  One workgroup barrier per chunk, none per K step.
//  * NW waves per workgroup: KW of them split the K steps and NW / KW split the channels.
//    Splitting K means each activation fragment read from LDS feeds RW MFMAs of one wave and
//    no fragment is read twice; the KW partial sums are reduced through LDS at the end.
//  * A chunk holds S K steps of every wave and the weight ring NS = S * NSLOT steps, so a loop
//    body of NSLOT chunks visits every LDS slot and ring slot at a fixed position, and every
//    s_waitcnt vmcnt value is a compile-time constant.  Loads past the end are out-of-range
//    buffer reads (they return zero), so each iteration issues the same loads.
//  * Split-K across workgroups hands INT32 tiles off 16 bytes per lane (w8a8_splitk_finish);
//    plan mode and the epilogue are shared with w8a8_kernel.
//  * WL 2 is the W4A8 weight: packed INT4 fragments of 512 bytes (8 bytes per lane per K
//    step, w8a8_wop) that become INT8 operands holding 16 * q; the INT32 sums are shifted
//    right by 4 (exact) before the shared epilogue.
#pragma once
#include "w8a8.hpp"

namespace specq {

template <int MT, int RW, int KW, int S, int NSLOT, int NW>
struct W8A8WsCfg {
  static constexpr int CW = NW / KW;                  // waves along channels
  static constexpr int BM = MT * 16, BNW = RW * 16, BN = CW * BNW;
  static constexpr int KC = S * 64 * KW;              // bytes of K per activation chunk
  static constexpr int SLOT = BM * KC;                // LDS bytes per chunk
  static constexpr int P = NSLOT - 1;                 // chunks of activation DMA in flight
  static constexpr int DMA_TOTAL = BM * KC / 1024;    // 1 KB DMA instructions per chunk
  static constexpr int A_L = DMA_TOTAL / NW;          // ... per wave
  static constexpr int NS = S * NSLOT;                // weight ring slots
  static constexpr int D = NS - 1;                    // K steps of weights in flight
  static constexpr int RED = BM * BN * 4;             // one reduction slice
  static constexpr bool OK = S >= 1 && NSLOT >= 2 && NSLOT <= 6 && NW % KW == 0 && KC % 256 == 0 &&
                             DMA_TOTAL % NW == 0 && A_L >= 1 && NS * RW + NSLOT * A_L <= 63 &&
                             NSLOT * SLOT + 64 <= 160 * 1024 && (KW == 1 || RED <= SLOT);
};

// The kernel body.  `slot_ptr(std::integral_constant<int, i>)` returns activation slot i
// (i < NSLOT, at least SLOT bytes each, 16-byte aligned).  The slots are separate LDS
// variables: the compiler's wait-count pass can then tell that reads of one slot do not
// depend on the DMA still filling another.  Also inlined into the plan-mode launch that holds
// several tilings (w8a8_plan.hpp), which passes slots sized for its largest tiling.
template <int MT, int RW, int KW, int S, int NSLOT, int NW, int WL, class SlotPtr>
__device__ __forceinline__ void w8a8_ws_body(W8A8Params p, SlotPtr slot_ptr) {
  using C = W8A8WsCfg<MT, RW, KW, S, NSLOT, NW>;
  static_assert(C::OK, "unsupported W8A8 weight-stream tile");
  constexpr int CW = C::CW, BM = C::BM, BNW = C::BNW, BN = C::BN, KC = C::KC, A_L = C::A_L;
  constexpr int NS = C::NS, D = C::D, P = C::P, SLOT = C::SLOT;
  tl_mark(p.tl, p.tl_cap, 0);  // diagnostics build: workgroup start

  int mc, unit;
  if (!chunked_unit(p.m_chunks, p.n_tiles * p.splits, mc, unit)) return;
  int split, tile;  // tile: launch-wide (counters, partials)
  split_decode(unit, p.n_tiles, p.splits, tile, split);
  const int ltile = w8a8_select_member(p, tile);  // tile within its GEMM (weights, outputs)

  int M = p.M;
  if (p.plan != nullptr) M = min(max(p.plan[0], 0), p.m_grid);
  M = uniform(M);
  const int m0 = mc * BM;
  if (m0 >= M) return;

  const int lane = lane_id(), w = uniform(wave_id()), g = lane >> 4, r = lane & 15;
  const int cw = w % CW, kw = w / CW;
  const int n0 = ltile * BN + cw * BNW;  // first channel of this wave
  const int kb = split * p.k_range;
  const int ke = min(p.K, kb + p.k_range);
  const int nchunks = (ke - kb + KC - 1) / KC;
  // Row-major weights: rotate the chunk order per workgroup (INT32 sums do not depend on it).
  const int rot = WL == 0 ? (int)(((unsigned)tile * 5u + (unsigned)split * 3u) % (unsigned)nchunks) : 0;
  int ke_v = ke;
  asm volatile("" : "+v"(ke_v));

  // ---- Activation DMA.  Chunk c covers K [kc0, kc0 + KC), kc0 = kb + KC * ((c + rot) mod
  // nchunks).  DMA instruction q (wave w issues q = w, w + NW, ...) fills 256-byte block
  // b = q / (BM/4), rows 4 * (q % (BM/4)) + lane / 16, LDS slot lane % 16 with piece
  // (lane % 16) ^ (row % 16) of the block.  LDS image: [block][row][16 slots of 16 bytes].
  const int m_rows = min(BM, M - m0);
  const rsrc_t asrc = make_rsrc(p.A + (int64_t)m0 * p.lda, (uint32_t)((m_rows - 1) * p.lda + p.K));
  uint32_t dma_off[A_L];
  int dma_k[A_L];  // K offset of the lane's piece within the chunk
#pragma unroll
  for (int i = 0; i < A_L; ++i) {
    const int q = w + NW * i;
    const int b = q / (BM / 4), row = 4 * (q % (BM / 4)) + g;
    dma_k[i] = b * 256 + 16 * (r ^ (row & 15));
    dma_off[i] = row < m_rows ? (uint32_t)(row * p.lda + dma_k[i]) : kOOB;
  }
  auto chunk_k0 = [&](int c) {
    int cc = c + rot;
    cc = cc >= nchunks ? cc - nchunks : cc;
    return kb + cc * KC;
  };
  auto dma_chunk = [&](int c, uint8_t* slot) {
    const int kc0 = chunk_k0(c);
#pragma unroll
    for (int i = 0; i < A_L; ++i) {
      const bool ok = (c < nchunks) & (dma_off[i] != kOOB) & (kc0 + dma_k[i] < ke_v);
      dma16(asrc, slot + (w + NW * i) * 1024, oob_unless(ok, dma_off[i] + (uint32_t)kc0));
    }
  };

  // ---- Weight stream.  Wave-local step i belongs to chunk i / S; its step j = i % S of the
  // chunk is K step kw + KW * j of the chunk.
  using WFrag = W8A8WFrag<WL>;
  const int n_rows_w = uniform(max(0, min(BNW, p.N - n0)));
  rsrc_t wsrc;
  uint32_t wrow[RW];
  uint32_t sstride;
  if constexpr (WL == 0) {
    wsrc = make_rsrc(p.W + (int64_t)min(n0, p.N - 1) * p.ldw,
                     n_rows_w > 0 ? (uint32_t)((n_rows_w - 1) * p.ldw + p.K) : 0u);
#pragma unroll
    for (int i = 0; i < RW; ++i) wrow[i] = (i * 16 + r < n_rows_w) ? (uint32_t)((i * 16 + r) * p.ldw + g * 16) : kOOB;
    sstride = 64;
  } else {
    constexpr uint32_t FB = W8A8WFragBytes<WL>::value;  // bytes of one packed fragment
    const int ntiles = (p.N + 15) / 16;
    const int ksteps = (p.K + 63) / 64;
    wsrc = make_rsrc(p.W, (uint32_t)((size_t)ksteps * ntiles * FB));
#pragma unroll
    for (int i = 0; i < RW; ++i)
      wrow[i] = (n0 / 16 + i < ntiles) ? (uint32_t)((n0 / 16 + i) * FB + lane * (FB / 64)) : kOOB;
    sstride = (uint32_t)ntiles * FB;
  }
  auto w_issue = [&](int c, int j, WFrag (&slot)[RW]) {
    const int step = (chunk_k0(c) >> 6) + kw + KW * j;  // global K step of chunk c, step j
    const bool live = (c < nchunks) & (step * 64 + g * 16 < ke_v);
#pragma unroll
    for (int t = 0; t < RW; ++t) {
      const uint32_t off = oob_unless(live & (wrow[t] != kOOB), wrow[t] + (uint32_t)step * sstride);
      slot[t] = w8a8_wload<WL>(wsrc, off);
    }
  };

  const bool owner = kw == 0;
  W8A8EpiScales<MT, RW> es;
  es.load(p, M, m0, n0, owner & (p.splits == 1));

  v4i acc[RW][MT];
#pragma unroll
  for (int t = 0; t < RW; ++t)
#pragma unroll
    for (int u = 0; u < MT; ++u) acc[t][u] = v4i{0, 0, 0, 0};

  // Steady state, step i = c*S + j: at the top of chunk c the DMA of chunk c + P is issued
  // (into LDS slot (c + P) % NSLOT); each step issues the weights of step i + D into ring
  // slot (i + D) % NS and consumes step i.  The prologue issues the same sequence for the
  // steps before 0, so the loads issued after any given one are the same at every step and
  // every wait count below is a compile-time constant:
  //   after step i's weights:  D weight steps + NSLOT DMA groups (j < S-1) or P (j = S-1);
  //   after chunk c's DMA:     P*S weight steps + P-1 DMA groups.
  WFrag ring[NS][RW];
  static_for<0, S - 1>([&](auto sc) {
    constexpr int s = decltype(sc)::value;
    w_issue(0, s, ring[s]);
    __builtin_amdgcn_sched_barrier(0);
  });
  static_for<0, P>([&](auto vc) {
    constexpr int v = decltype(vc)::value;
    dma_chunk(v, slot_ptr(vc));
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, S>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      constexpr int i = v * S + S - 1 + j;  // weight step issued here
      w_issue(i / S, i % S, ring[i]);
      __builtin_amdgcn_sched_barrier(0);
    });
  });

  // Main loop: NSLOT chunks per iteration, so LDS slot (c % NSLOT) and ring slot (i % NS)
  // are compile-time inside the body.
  for (int c0 = 0; c0 < nchunks; c0 += NSLOT) {
    static_for<0, NSLOT>([&](auto cc_) __attribute__((always_inline)) {
      constexpr int cl = decltype(cc_)::value;
      const int c = c0 + cl;
      wait_vmcnt<P * S * RW + (P - 1) * A_L>();  // this wave's DMA of chunk c has landed
      wg_barrier_lds();  // ... every wave's has, and nobody reads slot (c + P) % NSLOT any more
      if constexpr (cl == 0) {
        if (c0 == 0) tl_mark(p.tl, p.tl_cap, 1);  // diagnostics build: first chunk landed
      }
      dma_chunk(c + P, slot_ptr(std::integral_constant<int, (cl + P) % NSLOT>{}));
      __builtin_amdgcn_sched_barrier(0);
      const uint8_t* aslot = slot_ptr(cc_);
      static_for<0, S>([&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        constexpr int ri = (cl * S + j) % NS;           // ring slot of step i
        constexpr int rn = (cl * S + j + D) % NS;       // ring slot of step i + D
        constexpr int jn = (j + D) % S;                 // step i + D: step jn of chunk ...
        constexpr int cn = (j + D) / S;                 // ... c + cn
        w_issue(c + cn, jn, ring[rn]);
        __builtin_amdgcn_sched_barrier(0);
        constexpr int after = D * RW + (j < S - 1 ? NSLOT : P) * A_L;
        wait_vmcnt<after>();
        const int ks = kw + KW * j;  // K step within the chunk
        const int blk = ks >> 2, piece = 4 * (ks & 3) + g;
        v4i af[MT];
#pragma unroll
        for (int u = 0; u < MT; ++u) {
          const int row = u * 16 + r;
          af[u] = *reinterpret_cast<const v4i*>(aslot + (blk * BM + row) * 256 + 16 * (piece ^ r));
        }
#pragma unroll
        for (int a = 0; a < RW; ++a) {
          const v4i wf = w8a8_wop(ring[ri][a]);
#pragma unroll
          for (int u = 0; u < MT; ++u)
            acc[a][u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf, af[u], acc[a][u], 0, 0, 0);
        }
      });
    });
  }
  wait_vmcnt<0>();
  wg_barrier_lds();  // every wave is done with the activation slots
  tl_mark(p.tl, p.tl_cap, 2);  // diagnostics build: main loop done
  if constexpr (WL == 2) w8a8_unscale16(acc);

  // Reduce the KW waves of each channel group through LDS: every non-owner wave writes its
  // slice into its own activation slot (up to NSLOT slices per round), then the owner adds
  // them, so KW = 4 takes one round and two barriers.
  if constexpr (KW > 1) {
    constexpr int PR = KW - 1 < NSLOT ? KW - 1 : NSLOT;  // slices per round
    static_for<0, (KW - 1 + PR - 1) / PR>([&](auto rc) {
      constexpr int q0 = 1 + decltype(rc)::value * PR;
      static_for<0, PR>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        if (q0 + j < KW && kw == q0 + j) {
          int32_t* red = reinterpret_cast<int32_t*>(slot_ptr(jc));
#pragma unroll
          for (int a = 0; a < RW; ++a)
#pragma unroll
            for (int u = 0; u < MT; ++u)
              *reinterpret_cast<v4i*>(red + (u * 16 + r) * BN + cw * BNW + a * 16 + 4 * g) = acc[a][u];
        }
      });
      wg_barrier_lds();
      if (owner) {
        static_for<0, PR>([&](auto jc) {
          constexpr int j = decltype(jc)::value;
          if constexpr (q0 + j < KW) {
            const int32_t* red = reinterpret_cast<const int32_t*>(slot_ptr(jc));
#pragma unroll
            for (int a = 0; a < RW; ++a)
#pragma unroll
              for (int u = 0; u < MT; ++u)
                acc[a][u] += *reinterpret_cast<const v4i*>(red + (u * 16 + r) * BN + cw * BNW + a * 16 + 4 * g);
          }
        });
      }
      if constexpr (q0 + PR < KW) wg_barrier_lds();  // the next round reuses the slots
    });
  }

  const int cidx = mc * p.n_tiles + tile;
  if (p.splits == 1) {
    // The fp16 tile goes through LDS (row-major, 16-byte pieces XOR-swizzled by row), so that
    // each lane then stores 16 contiguous bytes of an output row and a wave's store covers
    // whole rows of the tile instead of 32-byte pieces of 16 rows.
    constexpr int PIECES = BN / 8;  // 16-byte pieces per tile row
    static_assert(BM * BN * 2 <= SLOT, "the fp16 tile fits one activation slot");
    uint8_t* ctile = slot_ptr(std::integral_constant<int, 0>{});
    if constexpr (KW > 1) wg_barrier_lds();  // the owners have read the reduction slices
    if (owner) {
#pragma unroll
      for (int a = 0; a < RW; ++a)
#pragma unroll
        for (int u = 0; u < MT; ++u) {
          const int row = u * 16 + r, nl = cw * BNW + a * 16 + 4 * g;
          const int pc = (nl >> 3) ^ (row & (PIECES - 1));
          *reinterpret_cast<v4h*>(ctile + row * (BN * 2) + pc * 16 + (nl & 4) * 2) = w8a8_cvt4(acc[a][u], es.a[u], es.w[a]);
        }
    }
    wg_barrier_lds();
    const int nt0 = ltile * BN;
    const bool v16 = ((uintptr_t)p.C % 16 == 0) & (p.ldc % 8 == 0);
    constexpr int NT = NW * 64, QN = BM * PIECES;
#pragma unroll
    for (int i = 0; i < (QN + NT - 1) / NT; ++i) {
      const int q = (int)threadIdx.x + i * NT;
      const int row = q / PIECES, pc = q % PIECES;
      const int m = m0 + row, n = nt0 + pc * 8;
      if ((QN % NT == 0 || q < QN) && m < M && n < p.N) {
        const v8h v = *reinterpret_cast<const v8h*>(ctile + row * (BN * 2) + ((pc ^ (row & (PIECES - 1))) * 16));
        _Float16* dst = reinterpret_cast<_Float16*>(p.C + (int64_t)m * p.ldc + n);
        if (v16 && n + 7 < p.N) {
          *reinterpret_cast<v8h*>(dst) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (n + e < p.N) dst[e] = v[e];
        }
      }
    }
    tl_mark(p.tl, p.tl_cap, 3);          // diagnostics build: stores issued
    tl_mark_drained(p.tl, p.tl_cap, 4);  // ... and completed
    return;
  }
  const rsrc_t prs = w8a8_partials_rsrc<BM, BN>(p, cidx);
  if (owner) {
#pragma unroll
    for (int a = 0; a < RW; ++a)
#pragma unroll
      for (int u = 0; u < MT; ++u)
        w8a8_publish_quad<BM, BN>(prs, split, u * 16 + r, cw * BNW + a * 16 + 4 * g, acc[a][u]);
  }
  tl_mark(p.tl, p.tl_cap, 3);  // diagnostics build: partials issued
  __shared__ int s_last_ws;
  w8a8_splitk_finish<BM, BN, NW * 64>(p, prs, cidx, m0, ltile * BN, M, &s_last_ws);
  tl_mark_drained(p.tl, p.tl_cap, 4);  // diagnostics build: hand-off (and, if last, the sum) done
}

template <int MT, int RW, int KW, int S, int NSLOT, int NW, int WL>
__global__ __launch_bounds__(NW * 64) void w8a8_ws_kernel(W8A8Params p) {
  constexpr int SLOT = W8A8WsCfg<MT, RW, KW, S, NSLOT, NW>::SLOT;
  __shared__ __attribute__((aligned(16))) uint8_t lds_s0[SLOT], lds_s1[SLOT];
  __shared__ __attribute__((aligned(16))) uint8_t lds_s2[NSLOT > 2 ? SLOT : 16], lds_s3[NSLOT > 3 ? SLOT : 16];
  __shared__ __attribute__((aligned(16))) uint8_t lds_s4[NSLOT > 4 ? SLOT : 16], lds_s5[NSLOT > 5 ? SLOT : 16];
  w8a8_ws_body<MT, RW, KW, S, NSLOT, NW, WL>(p, [&](auto ic) -> uint8_t* {
    constexpr int i = decltype(ic)::value;
    if constexpr (i == 0) return lds_s0;
    else if constexpr (i == 1) return lds_s1;
    else if constexpr (i == 2) return lds_s2;
    else if constexpr (i == 3) return lds_s3;
    else if constexpr (i == 4) return lds_s4;
    else return lds_s5;
  });
}

}  // namespace specq
