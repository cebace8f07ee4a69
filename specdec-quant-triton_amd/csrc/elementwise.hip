// Elementwise steps that sit between the GEMMs of a verification layer, plus their C ABI:
//   silu_mul            h = fp16(silu(gate) * up)                        (fp32 math)
//   quantize_act_int8   per-token symmetric INT8 (kernels.py:58-62 on the device)
//   silu_mul_quant_int8 the two fused: the fp16 h is formed in registers and quantised
//                       without a round trip through HBM.
// One workgroup per token row; rows at or beyond the active M (plan[0] in plan mode) exit.
// Fast path (16-byte aligned rows, N a multiple of 8, N <= 32768): each thread issues all of
// its 16-byte loads of the row at once and keeps the row in registers between the amax pass
// and the quantise pass, so a row costs one memory round trip instead of one per loop
// iteration.  Other shapes use the element-wise loop.
// The quantiser reproduces the reference formula bit for bit: amax in fp32,
// s = max(amax, 1e-8) / 127 (IEEE division), q = clamp(rne(x / s), -127, 127).
#include "api_common.hpp"
#include "common.hpp"

namespace specq {

struct EltParams {
  const _Float16* x; int64_t ldx;    // quantize input, or gate
  const _Float16* up; int64_t ld_up; // silu_mul only
  _Float16* h; int64_t ldh;          // silu_mul output
  int8_t* q; int64_t ldq; float* s;  // quantize outputs
  const int32_t* plan;
  int M, N, m_grid;
};

// silu(x) = x / (1 + e^-x) from the hardware base-2 exponential and reciprocal (about 1 ulp
// each; with the rounding of x * log2(e) the fp32 result is within ~2^-19 relative of the
// exact value for |x| up to fp16's range, far below the fp16 rounding that follows).  Large
// negative x gives e^-x = inf and a reciprocal of 0, so silu = -0 as in the exact form.
__device__ __forceinline__ float silu_f(float x) {
  const float e = __builtin_amdgcn_exp2f(-x * 1.44269504088896341f);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}
// silu(gate) * up is rounded to fp32 and then cast to fp16 (f32_opaque keeps the multiply and
// the cast from being fused into one v_fma_mix with a single rounding).

template <int MODE>  // 0 = silu_mul, 1 = quantize, 2 = silu_mul + quantize
__global__ __launch_bounds__(256) void elt_kernel(EltParams p) {
  int M = p.M;
  if (p.plan != nullptr) M = min(max(p.plan[0], 0), p.m_grid);
  const int m = blockIdx.x;
  if (m >= uniform(M)) return;
  const _Float16* xr = p.x + (int64_t)m * p.ldx;
  const _Float16* ur = (MODE != 1) ? p.up + (int64_t)m * p.ld_up : nullptr;
  const int N = p.N;

  auto value = [&](int k) -> _Float16 {
    if constexpr (MODE == 1) return xr[k];
    else return (_Float16)f32_opaque(silu_f((float)xr[k]) * (float)ur[k]);
  };

  if constexpr (MODE == 0) {
    _Float16* hr = p.h + (int64_t)m * p.ldh;
    for (int k = threadIdx.x; k < N; k += blockDim.x) hr[k] = value(k);
    return;
  } else {
    __shared__ float red[256 / kWave];
    float amax = 0.f;
    for (int k = threadIdx.x; k < N; k += blockDim.x) amax = fmaxf(amax, fabsf((float)value(k)));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    if (lane_id() == 0) red[wave_id()] = amax;
    __syncthreads();
    amax = red[0];
    for (int i = 1; i < (int)(blockDim.x / kWave); ++i) amax = fmaxf(amax, red[i]);
    const float s = fmaxf(amax, 1e-8f) / 127.0f;
    int8_t* qr = p.q + (int64_t)m * p.ldq;
    for (int k = threadIdx.x; k < N; k += blockDim.x) {
      float v = rintf((float)value(k) / s);
      v = fminf(fmaxf(v, -127.f), 127.f);
      qr[k] = (int8_t)v;
    }
    if (threadIdx.x == 0) p.s[m] = s;
  }
}

// Register-resident row: thread t holds the 8-element vectors t, t + NT, ... (VPT of them).
// Wide rows run NT = 1024 threads (four waves per SIMD hide the exp / reciprocal chains).
template <int MODE, int VPT, int NT>
__global__ __launch_bounds__(NT) void elt_vec_kernel(EltParams p) {
  int M = p.M;
  if (p.plan != nullptr) M = min(max(p.plan[0], 0), p.m_grid);
  const int m = blockIdx.x;
  if (m >= uniform(M)) return;
  const int nv = p.N / 8, t = threadIdx.x;
  const v8h* xr = reinterpret_cast<const v8h*>(p.x + (int64_t)m * p.ldx);
  const v8h* ur = MODE != 1 ? reinterpret_cast<const v8h*>(p.up + (int64_t)m * p.ld_up) : nullptr;
  v8h xv[VPT], uv[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int v = t + NT * i;
    if (v < nv) {
      xv[i] = xr[v];
      if constexpr (MODE != 1) uv[i] = ur[v];
    }
  }
  v8h val[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (MODE == 1) val[i][j] = xv[i][j];
      else val[i][j] = (_Float16)f32_opaque(silu_f((float)xv[i][j]) * (float)uv[i][j]);
    }
  if constexpr (MODE == 0) {
    v8h* hr = reinterpret_cast<v8h*>(p.h + (int64_t)m * p.ldh);
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      if (t + NT * i < nv) hr[t + NT * i] = val[i];
    return;
  } else {
    __shared__ float red[NT / kWave];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      if (t + NT * i < nv)
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf((float)val[i][j]));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    if (lane_id() == 0) red[wave_id()] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int i = 1; i < NT / kWave; ++i) amax = fmaxf(amax, red[i]);
    const float s = fmaxf(amax, 1e-8f) / 127.0f;
    v2i* qr = reinterpret_cast<v2i*>(p.q + (int64_t)m * p.ldq);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      if (t + NT * i >= nv) continue;
      int w[2] = {0, 0};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float v = rintf((float)val[i][j] / s);
        v = fminf(fmaxf(v, -127.f), 127.f);
        w[j >> 2] |= ((int)v & 0xff) << (8 * (j & 3));
      }
      qr[t + NT * i] = v2i{w[0], w[1]};
    }
    if (t == 0) p.s[m] = s;
  }
}

template <int MODE>
static const void* elt_vec_fn(int vpt, int nt) {
  if (nt == 1024) {
    switch (vpt) {
      case 1: return reinterpret_cast<const void*>(&elt_vec_kernel<MODE, 1, 1024>);
      case 2: return reinterpret_cast<const void*>(&elt_vec_kernel<MODE, 2, 1024>);
      case 4: return reinterpret_cast<const void*>(&elt_vec_kernel<MODE, 4, 1024>);
    }
    return nullptr;
  }
  switch (vpt) {
    case 1: return reinterpret_cast<const void*>(&elt_vec_kernel<MODE, 1, 256>);
    case 2: return reinterpret_cast<const void*>(&elt_vec_kernel<MODE, 2, 256>);
    case 4: return reinterpret_cast<const void*>(&elt_vec_kernel<MODE, 4, 256>);
    case 8: return reinterpret_cast<const void*>(&elt_vec_kernel<MODE, 8, 256>);
    case 16: return reinterpret_cast<const void*>(&elt_vec_kernel<MODE, 16, 256>);
  }
  return nullptr;
}

static int launch_elt(int mode, EltParams& p, hipStream_t stream) {
  const int m_grid = p.m_grid;
  if (m_grid == 0) return SPECQ_OK;
  // Vector path: 16-byte aligned fp16 rows, 8-byte aligned int8 rows, N a multiple of 8.
  bool vec = p.N % 8 == 0 && p.N <= 16 * 8 * 256 && (uintptr_t)p.x % 16 == 0 && p.ldx % 8 == 0;
  if (mode != 1) vec = vec && (uintptr_t)p.up % 16 == 0 && p.ld_up % 8 == 0;
  if (mode == 0) vec = vec && (uintptr_t)p.h % 16 == 0 && p.ldh % 8 == 0;
  else vec = vec && (uintptr_t)p.q % 8 == 0 && p.ldq % 8 == 0;
  const void* fn = nullptr;
  int nt = 256;
  if (vec) {
    nt = p.N / 8 >= 1024 ? 1024 : 256;
    const int per_thread = (p.N / 8 + nt - 1) / nt;
    int vpt = 1;
    while (vpt < per_thread) vpt <<= 1;
    fn = mode == 0 ? elt_vec_fn<0>(vpt, nt) : (mode == 1 ? elt_vec_fn<1>(vpt, nt) : elt_vec_fn<2>(vpt, nt));
  }
  if (fn == nullptr) {
    nt = 256;
    fn = mode == 0 ? reinterpret_cast<const void*>(&elt_kernel<0>)
       : mode == 1 ? reinterpret_cast<const void*>(&elt_kernel<1>)
                   : reinterpret_cast<const void*>(&elt_kernel<2>);
  }
  return launch(fn, m_grid, nt, 0, stream, &p);
}

}  // namespace specq

using namespace specq;

extern "C" int specq_silu_mul(const void* gate, int64_t ld_gate, const void* up, int64_t ld_up, void* h,
                              int64_t ld_h, int M, int N, int grid_m_max, const int32_t* plan, void* stream) {
  clear_error();
  SPECQ_REQUIRE(gate && up && h, SPECQ_EINVAL, "silu_mul: null tensor pointer");
  SPECQ_REQUIRE(M >= 0 && N > 0 && ld_gate >= N && ld_up >= N && ld_h >= N, SPECQ_EINVAL,
                "silu_mul: bad sizes or strides");
  SPECQ_REQUIRE(grid_m_max == 0 || grid_m_max >= M, SPECQ_EINVAL, "silu_mul: grid_m_max < M");
  EltParams p = {};
  p.x = (const _Float16*)gate; p.ldx = ld_gate; p.up = (const _Float16*)up; p.ld_up = ld_up;
  p.h = (_Float16*)h; p.ldh = ld_h; p.plan = plan; p.M = M; p.N = N; p.m_grid = grid_m_max > 0 ? grid_m_max : M;
  return launch_elt(0, p, (hipStream_t)stream);
}

extern "C" int specq_quantize_act_int8(const void* x, int64_t ldx, int8_t* q, int64_t ldq, float* s, int M, int K,
                                       int grid_m_max, const int32_t* plan, void* stream) {
  clear_error();
  SPECQ_REQUIRE(x && q && s, SPECQ_EINVAL, "quantize_act_int8: null tensor pointer");
  SPECQ_REQUIRE(M >= 0 && K > 0 && ldx >= K && ldq >= K, SPECQ_EINVAL, "quantize_act_int8: bad sizes or strides");
  SPECQ_REQUIRE(grid_m_max == 0 || grid_m_max >= M, SPECQ_EINVAL, "quantize_act_int8: grid_m_max < M");
  EltParams p = {};
  p.x = (const _Float16*)x; p.ldx = ldx; p.q = q; p.ldq = ldq; p.s = s; p.plan = plan;
  p.M = M; p.N = K; p.m_grid = grid_m_max > 0 ? grid_m_max : M;
  return launch_elt(1, p, (hipStream_t)stream);
}

extern "C" int specq_silu_mul_quant_int8(const void* gate, int64_t ld_gate, const void* up, int64_t ld_up, int8_t* q,
                                         int64_t ldq, float* s, int M, int N, int grid_m_max, const int32_t* plan,
                                         void* stream) {
  clear_error();
  SPECQ_REQUIRE(gate && up && q && s, SPECQ_EINVAL, "silu_mul_quant_int8: null tensor pointer");
  SPECQ_REQUIRE(M >= 0 && N > 0 && ld_gate >= N && ld_up >= N && ldq >= N, SPECQ_EINVAL,
                "silu_mul_quant_int8: bad sizes or strides");
  SPECQ_REQUIRE(grid_m_max == 0 || grid_m_max >= M, SPECQ_EINVAL, "silu_mul_quant_int8: grid_m_max < M");
  EltParams p = {};
  p.x = (const _Float16*)gate; p.ldx = ld_gate; p.up = (const _Float16*)up; p.ld_up = ld_up;
  p.q = q; p.ldq = ldq; p.s = s; p.plan = plan; p.M = M; p.N = N; p.m_grid = grid_m_max > 0 ? grid_m_max : M;
  return launch_elt(2, p, (hipStream_t)stream);
}
