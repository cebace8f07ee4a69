// Shared device helpers for the gfx950 (MI355X, CDNA4) quantized verification kernels.
//
// Everything here is written for 64-wide wavefronts and the CDNA4 MFMA lane layouts:
//   16x16xK MFMA : operand lane l holds row (l % 16) and the K-slice group (l / 16);
//                  result lane l holds column (l % 16), rows 4*(l/16) + i, i = 0..3.
// Because a dot product is invariant under a permutation of K applied to both operands,
// the kernels are free to choose which global K indices a lane's operand bytes hold, as
// long as the A- and B-operand loads use the same mapping.  They use that freedom to make
// every lane load long contiguous runs straight from HBM into VGPRs.
#pragma once
#include <type_traits>
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace specq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / kWave; }

// Read a value that is uniform across the workgroup into an SGPR.
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// ---------------------------------------------------------------------------------------
// Raw buffer loads with hardware range checking.
//
// A buffer resource covers one workgroup's slab of a matrix (num_records bytes from its
// first row).  Lanes whose offset is >= num_records read zeros, so rows past the end of the
// matrix and K positions past the end of a row are masked without branches: the masked lane
// is handed the offset kOOB.  Keeping loads free of control flow lets the compiler count
// outstanding loads exactly (vmcnt), which is what makes register double-buffering work.
// ---------------------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOOB = 0x80000000u;
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer descriptor (32-bit data format)

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t num_records) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)num_records, kRsrcWord3);
}

// 16 bytes at row_off + k of the slab; VEC-byte pieces at or beyond kend read as zero.
template <int VEC>
__device__ __forceinline__ v4i bload16(rsrc_t rs, uint32_t row_off, int k, int kend) {
  if constexpr (VEC == 16) {
    return __builtin_amdgcn_raw_buffer_load_b128(rs, k < kend ? row_off + k : kOOB, 0, 0);
  } else if constexpr (VEC == 8) {
    const auto lo = __builtin_amdgcn_raw_buffer_load_b64(rs, k < kend ? row_off + k : kOOB, 0, 0);
    const auto hi = __builtin_amdgcn_raw_buffer_load_b64(rs, k + 8 < kend ? row_off + k + 8 : kOOB, 0, 0);
    return v4i{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};
  } else if constexpr (VEC == 4) {
    v4i r;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      r[i] = (int)__builtin_amdgcn_raw_buffer_load_b32(rs, k + 4 * i < kend ? row_off + k + 4 * i : kOOB, 0, 0);
    return r;
  } else {
    int w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int b = __builtin_amdgcn_raw_buffer_load_b8(rs, k + i < kend ? row_off + k + i : kOOB, 0, 0);
      w[i >> 2] |= (b & 0xff) << (8 * (i & 3));
    }
    return v4i{w[0], w[1], w[2], w[3]};
  }
}

// ---------------------------------------------------------------------------------------
// 16-byte operand loads with K-tail masking at VEC-byte granularity.
// VEC is the largest power of two (<=16) dividing K, the row stride and the base pointer,
// so a VEC chunk is either entirely inside [0, K) or entirely outside it.
// ---------------------------------------------------------------------------------------
template <int VEC>
__device__ __forceinline__ v4i load16_masked(const int8_t* row, int k, int K) {
  v4i r = {0, 0, 0, 0};
  if constexpr (VEC == 16) {
    if (k < K) r = *reinterpret_cast<const v4i*>(row + k);
  } else if constexpr (VEC == 8) {
    v2i lo = {0, 0}, hi = {0, 0};
    if (k < K) lo = *reinterpret_cast<const v2i*>(row + k);
    if (k + 8 < K) hi = *reinterpret_cast<const v2i*>(row + k + 8);
    r.x = lo.x; r.y = lo.y; r.z = hi.x; r.w = hi.y;
  } else if constexpr (VEC == 4) {
    const int* p = reinterpret_cast<const int*>(row + k);
    if (k < K) r.x = p[0];
    if (k + 4 < K) r.y = p[1];
    if (k + 8 < K) r.z = p[2];
    if (k + 12 < K) r.w = p[3];
  } else {
    int w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      int b = (k + i < K) ? (int)(uint8_t)row[k + i] : 0;
      w[i >> 2] |= b << (8 * (i & 3));
    }
    r.x = w[0]; r.y = w[1]; r.z = w[2]; r.w = w[3];
  }
  return r;
}

// ---------------------------------------------------------------------------------------
// int8 / int4 -> fp16 conversions by exponent injection (exact for the ranges used).
// 0x64 in the high byte of an fp16 gives 1024 + (low byte), with a unit ulp on [1024, 2048).
// ---------------------------------------------------------------------------------------

// Four signed int8 in a dword -> two packed half2 (bytes 0,1 -> lo; bytes 2,3 -> hi).
__device__ __forceinline__ void i8x4_to_h2x2(uint32_t x, v2h& lo, v2h& hi) {
  uint32_t u = x ^ 0x80808080u;  // signed -> biased unsigned (x + 128)
  // v_perm_b32(s0, s1, sel): byte selector 0..3 picks from s1, 4..7 from s0.
  uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // [b0, 0x64, b1, 0x64]
  uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // [b2, 0x64, b3, 0x64]
  const v2h bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  lo = __builtin_bit_cast(v2h, a) - bias;
  hi = __builtin_bit_cast(v2h, b) - bias;
}

// Eight signed int8 (two dwords) -> v8h.
__device__ __forceinline__ v8h i8x8_to_h8(uint32_t x0, uint32_t x1) {
  v2h a, b, c, d;
  i8x4_to_h2x2(x0, a, b);
  i8x4_to_h2x2(x1, c, d);
  v8h r;
  r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
  r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
  return r;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------------------
// Cross-workgroup hand-off without cache-wide fences.
//
// A split reduction publishes partial results that the last workgroup to arrive combines.
// An agent-scope release/acquire fence would write back and invalidate the whole L2 of the
// XCD (buffer_wbl2 / buffer_inv), which serialises across the XCD's workgroups and costs
// microseconds per call.  Instead every published value is written with an agent-scope
// atomic store (coherent at device scope, so nothing dirty stays behind in a non-coherent
// cache), the writer waits until those stores have completed (s_waitcnt vmcnt(0)) before it
// increments the arrival counter, and the consumer reads the values with agent-scope atomic
// loads after observing the final count.  This is the ordering the compiler's memory model
// produces for release/acquire, without the cache-wide maintenance that is only needed for
// ordinary (non-atomic) data.
// ---------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void publish(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T collect(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The same hand-off, 16 bytes per lane: buffer stores and loads carrying the cache-coherence
// bit (SC1) that the compiler puts on relaxed agent-scope atomic stores and loads, so whole
// int32x4 / float4 partial tiles move in one instruction per lane instead of four.
constexpr int kAuxAgent = 16;  // SC1
__device__ __forceinline__ void publish16(rsrc_t rs, uint32_t off, v4i v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, 0, kAuxAgent);
}
__device__ __forceinline__ v4i collect16(rsrc_t rs, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kAuxAgent);
}
// All of this wave's outstanding memory operations have completed.
// s_waitcnt with vmcnt = N (expcnt and lgkmcnt left at their maximum, i.e. not waited on).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Buffer offset `off`, or out of range (reads as zero) when !ok.  Bit 31 is set arithmetically
// rather than selected: offsets here are < 2^31, and a select on a cheap-to-skip address tends
// to be turned into a branch around the load, which costs a vmcnt(0) at the join.
__device__ __forceinline__ uint32_t oob_unless(bool ok, uint32_t off) { return off | ((uint32_t)(!ok) << 31); }

// Returns x unchanged while hiding from the compiler how it was computed.  Used on an fp32
// product that is then cast to fp16: the compiler otherwise folds fptrunc(a * b) into one
// v_fma_mix, which rounds the exact product to fp16 once instead of rounding to fp32 first
// (the two differ when the fp32 product lands on an fp16 rounding midpoint).
__device__ __forceinline__ float f32_opaque(float x) {
  asm("" : "+v"(x));
  return x;
}

// 16-byte LDS DMA (buffer_load_dwordx4 ... lds): lane l's 16 bytes from voff land at
// lds_frag + 16*l (lds_frag must be wave-uniform); out-of-range lanes write zeros.
__device__ __forceinline__ void dma16(rsrc_t rs, uint8_t* lds_frag, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)lds_frag, 16, voff, 0, 0, 0);
}

// Workgroup barriers for software pipelines.  __syncthreads() is a workgroup fence plus
// s_barrier, and the fence waits for every outstanding load (vmcnt(0)), which drains a
// prefetch pipeline at each barrier.  These issue s_barrier with compiler-only fences:
//  * wg_barrier(): orders nothing in hardware; for data the waves made visible themselves
//    (e.g. LDS DMA completed with an explicit s_waitcnt vmcnt before the barrier).
//  * wg_barrier_lds(): first waits for this wave's LDS operations (lgkmcnt(0)), so LDS
//    writes before it are visible to every wave after it and LDS reads before it are done.
__device__ __forceinline__ void wg_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ void wait_lgkm0() {
  // s_waitcnt encoding: vmcnt 63 (no wait), expcnt 7 (no wait), lgkmcnt 0.
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ void wg_barrier_lds() {
  wait_lgkm0();
  wg_barrier();
}

// Per-workgroup timestamps, compiled only into the diagnostics build of the library
// (-DSPECQ_DIAG, libspecq_diag.so): thread 0 of workgroup b stores s_memrealtime (a 100 MHz
// clock) at tl[b * kTlMarks + i] with an ordinary vector store.  In the product build the
// kernels' tl pointer stays null and this compiles to nothing.
constexpr int kTlMarks = 16;
__device__ __forceinline__ void tl_mark(uint64_t* tl, int cap, int i) {
#ifdef SPECQ_DIAG
  if (tl != nullptr && threadIdx.x == 0 && (int)blockIdx.x < cap)
    tl[(int64_t)blockIdx.x * kTlMarks + i] = __builtin_amdgcn_s_memrealtime();
#else
  (void)tl; (void)cap; (void)i;
#endif
}
// The same from lane 0 of every wave: wave w writes mark i + w (marks 8.. hold per-wave times).
__device__ __forceinline__ void tl_mark_wave(uint64_t* tl, int cap, int i) {
#ifdef SPECQ_DIAG
  if (tl != nullptr && (threadIdx.x & 63) == 0 && (int)blockIdx.x < cap)
    tl[(int64_t)blockIdx.x * kTlMarks + i + (int)(threadIdx.x >> 6)] = __builtin_amdgcn_s_memrealtime();
#else
  (void)tl; (void)cap; (void)i;
#endif
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Workgroup id -> (M-chunk mc, work unit): chunk-major, id = mc * units + unit.  In plan mode
// the grid covers the largest M while the active M usually fills only the first chunks; the
// workgroups of those chunks then come first in dispatch order, and the trailing ones (which
// only read the plan and exit) do not hold up the dispatch of active ones behind them.
__device__ __forceinline__ bool chunked_unit(int m_chunks, int units, int& mc, int& unit) {
  const int id = blockIdx.x;
  mc = id / units;
  unit = id - mc * units;
  return mc < m_chunks;
}
__host__ __device__ inline int chunked_grid(int units, int m_chunks) { return units * m_chunks; }
// The same grid with the M-chunks of a unit 8 workgroups apart, in blocks of 8 units (a
// trailing partial block runs its units' chunks back to back): the chunks of one channel tile
// share blockIdx.x mod 8 -- the XCD the dispatcher deals them to -- and run at the same time, so
// the weight lines the first chunk reads from memory reach the other chunks from that XCD's L2.
__device__ __forceinline__ bool interleaved_unit(int m_chunks, int units, int& mc, int& unit) {
  const int id = blockIdx.x;
  const int full = (units / 8) * 8;
  if (id < full * m_chunks) {
    const int blk = id / (8 * m_chunks), rem = id - blk * (8 * m_chunks);
    mc = rem / 8;
    unit = blk * 8 + rem % 8;
    return true;
  }
  const int rem = id - full * m_chunks, tail = units - full;
  if (tail <= 0 || rem >= tail * m_chunks) return false;
  mc = rem / tail;
  unit = full + rem % tail;
  return true;
}

// Channel tile and split-K index of chunk-local unit `unit` (n_tiles tiles x splits).  The
// splits of a tile are placed 8 units apart, in blocks of 8 tiles x splits units (the tiles of a
// trailing partial block run their splits back to back), so the workgroups of one tile share
// blockIdx.x mod 8 -- the XCD the dispatcher deals them to -- and the workgroups running next to
// each other in dispatch order cover different tiles.  Measured on the split-K launches of the
// Llama-3-8B linears: the device-coherent stores of the partial tiles complete in 0.4-0.6 us
// instead of 0.9-1.4 us when neighbouring workgroups are the splits of one tile (W4A16 q|k|v at
// M = 72: 19.3 -> 16.3 us per launch).  The result does not depend on the order.
__device__ __forceinline__ void split_decode(int unit, int n_tiles, int splits, int& tile, int& split) {
  if (splits == 1) {
    tile = unit;
    split = 0;
    return;
  }
  constexpr int X = 8;
  const int full = (n_tiles / X) * X;
  if (unit < full * splits) {
    const int blk = unit / (X * splits), r = unit - blk * (X * splits);
    tile = blk * X + r % X;
    split = r / X;
    return;
  }
  const int r = unit - full * splits;
  tile = full + r / splits;
  split = r % splits;
}

__device__ __forceinline__ void wait_all_memory() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Diagnostics build: mark i once every memory operation this wave issued has completed
// (thread 0's wave: in the kernels below that is the wave whose stores finish the tile).
__device__ __forceinline__ void tl_mark_drained(uint64_t* tl, int cap, int i) {
#ifdef SPECQ_DIAG
  wait_all_memory();
  tl_mark(tl, cap, i);
#else
  (void)tl; (void)cap; (void)i;
#endif
}

// Called by every thread after the workgroup's publish() calls: returns true in the last
// workgroup to arrive (of `expected`) at counter `ctr`, which is then reset to zero.
// The caller reads the published values with collect() only when this returns true.
__device__ __forceinline__ bool arrive_last(int32_t* ctr, int expected, int* s_flag, uint64_t* tl = nullptr,
                                            int tl_cap = 0) {
  wait_all_memory();
  tl_mark(tl, tl_cap, 5);  // diagnostics build: this wave's published values acknowledged
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = (prev == expected - 1);
    if (last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = last;
  }
  __syncthreads();
  tl_mark(tl, tl_cap, 6);  // diagnostics build: the arrival count has come back
  const bool last = *s_flag != 0;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return last;
}

}  // namespace specq
