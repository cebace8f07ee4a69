// Measurement helpers of the diagnostics build (libspecq_diag.so, compiled with -DSPECQ_DIAG).
//
// The product library compiles only diag_timeline() from this file, which then always reports
// "no timeline", so its kernels never write timestamps.  The diagnostics build adds:
//  * specq_diag_set_timeline: a device buffer of [cap][kTlMarks] uint64 into which every
//    following W8A8 and attention launch writes per-workgroup s_memrealtime marks (kernel
//    start, first operand data landed, main loop done, stores issued, all memory done);
//  * specq_diag_stream_read: a plain streaming read of a buffer (16-byte loads, XOR-reduced),
//    the floor a weight-streaming GEMM launch of the same bytes is measured against;
//  * specq_diag_xcc_ids: the XCD (hardware register XCC_ID) each workgroup of a launch ran on,
//    which shows how the dispatcher deals workgroups to the XCDs.
#include <atomic>

#include "api_common.hpp"
#include "common.hpp"

namespace specq {

static std::atomic<uint64_t*> g_tl{nullptr};
static std::atomic<int> g_tl_cap{0};

void diag_timeline(uint64_t** tl, int* cap) {
  *tl = g_tl.load();
  *cap = *tl ? g_tl_cap.load() : 0;
}

#ifdef SPECQ_DIAG
// Workgroup b reads bytes [b * per_wg, (b + 1) * per_wg) of buf, each wave U 1 KB pieces in
// flight per round, and keeps an XOR of everything it read; the sink is written only if that
// XOR takes an impossible value, so the loads cannot be removed and nothing else is stored.
template <int U>
__global__ __launch_bounds__(512) void diag_stream_read_kernel(const int8_t* buf, int64_t per_wg, int64_t total,
                                                               int* sink) {
  const int lane = lane_id(), w = wave_id(), nw = blockDim.x / kWave;
  const int64_t base = (int64_t)blockIdx.x * per_wg;
  const int64_t end = base + per_wg < total ? base + per_wg : total;
  v4i acc = {0, 0, 0, 0};
  for (int64_t off = base + ((int64_t)w * U) * 1024 + lane * 16; off < end; off += (int64_t)nw * U * 1024) {
    v4i t[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t o = off + (int64_t)u * 1024;
      t[u] = o < end ? *reinterpret_cast<const v4i*>(buf + o) : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= t[u];
  }
  const int x = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (x == 0x7e57c0de && lane == 63) sink[blockIdx.x] = x;
}

__global__ void diag_xcc_kernel(int* out) {
  int x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(x));
  if (threadIdx.x == 0) out[blockIdx.x] = x;
}
#endif

}  // namespace specq

#ifdef SPECQ_DIAG
extern "C" int specq_diag_set_timeline(void* tl, int cap) {
  specq::clear_error();
  if (tl != nullptr && cap <= 0) return specq::fail(SPECQ_EINVAL, "diag_set_timeline: cap must be positive");
  specq::g_tl_cap.store(tl ? cap : 0);
  specq::g_tl.store(reinterpret_cast<uint64_t*>(tl));
  return SPECQ_OK;
}

extern "C" int specq_diag_stream_read(const void* buf, int64_t bytes, int wgs, int waves, int unroll, int* sink,
                                      void* stream) {
  specq::clear_error();
  SPECQ_REQUIRE(buf && sink && bytes > 0 && bytes % 16 == 0 && (uintptr_t)buf % 16 == 0, SPECQ_EINVAL,
                "diag_stream_read: 16-byte aligned buffer of a positive multiple of 16 bytes required");
  SPECQ_REQUIRE(wgs >= 1 && wgs <= 65536 && (waves == 4 || waves == 8), SPECQ_EINVAL,
                "diag_stream_read: 1..65536 workgroups of 4 or 8 waves");
  const int64_t per_wg = specq::ceil_div64(specq::ceil_div64(bytes, wgs), 1024) * 1024;
  const void* fn = nullptr;
  switch (unroll) {
    case 2: fn = (const void*)&specq::diag_stream_read_kernel<2>; break;
    case 4: fn = (const void*)&specq::diag_stream_read_kernel<4>; break;
    case 8: fn = (const void*)&specq::diag_stream_read_kernel<8>; break;
    case 16: fn = (const void*)&specq::diag_stream_read_kernel<16>; break;
    default: return specq::fail(SPECQ_EINVAL, "diag_stream_read: unroll must be 2, 4, 8 or 16");
  }
  const int8_t* b = reinterpret_cast<const int8_t*>(buf);
  void* args[] = {&b, const_cast<int64_t*>(&per_wg), &bytes, &sink};
  hipError_t e = hipLaunchKernel(fn, dim3(wgs), dim3(waves * 64), args, 0, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return specq::fail(SPECQ_EIO, "diag_stream_read: launch failed");
  return SPECQ_OK;
}
#endif

#ifdef SPECQ_DIAG
// out[b] = XCD of workgroup b, for a launch of `wgs` workgroups of `threads` threads.
extern "C" int specq_diag_xcc_ids(int* out, int wgs, int threads, void* stream) {
  specq::clear_error();
  SPECQ_REQUIRE(out && wgs >= 1 && wgs <= (1 << 20) && threads >= 64 && threads <= 1024 && threads % 64 == 0,
                SPECQ_EINVAL, "diag_xcc_ids: 1..2^20 workgroups of 64..1024 threads");
  void* args[] = {&out};
  hipError_t e = hipLaunchKernel((const void*)&specq::diag_xcc_kernel, dim3(wgs), dim3(threads), args, 0,
                                 reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return specq::fail(SPECQ_EIO, "diag_xcc_ids: launch failed");
  return SPECQ_OK;
}
#endif
