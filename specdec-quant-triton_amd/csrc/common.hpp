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
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace specq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / kWave; }

// Read a value that is uniform across the workgroup into an SGPR.
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

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

}  // namespace specq
