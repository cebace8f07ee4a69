// Shared host-side pieces of the C ABI: thread-local error text, launch wrapper, device info,
// and the kernel-attribute query that dispatches to each kernel family.
#include <atomic>
#include <mutex>
#include <set>
#include <vector>

#include "api_common.hpp"
#include "tuned_tiles.hpp"

namespace specq {

// Measured table on (1) or off (0, the cost models only), through specq_set_option("tuned_tiles", v).
std::atomic<int> g_tuned_tiles{1};

bool tuned_tile(int kind, int N, int K, int M, int* block_m, int* block_n, int* split_k) {
  if (g_tuned_tiles.load() == 0 || device_cus() != 256 || M > 300) return false;
  // Steps of the table: 0 = M 1..8, 1 = M 9..16, r >= 2 = the 16 rows up to 16 r.
  const int step = M <= 8 ? 0 : (M + 15) / 16;
  for (int i = 0; i < kTunedTileCount; ++i) {
    const TunedTile& t = kTunedTiles[i];
    if (t.kind == kind && t.N == N && t.K == K && t.step == step) {
      *block_m = t.block_m;
      *block_n = t.block_n;
      *split_k = t.split_k;
      return true;
    }
  }
  return false;
}

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

int launch(const void* fn, int grid, int threads, size_t lds, hipStream_t stream, void* params) {
  if (grid <= 0) return SPECQ_OK;
  void* args[] = {params};
  hipError_t e = hipLaunchKernel(fn, dim3(grid), dim3(threads), args, lds, stream);
  if (e != hipSuccess) {
    set_error("hipLaunchKernel failed: %s (grid=%d threads=%d lds=%zu)", hipGetErrorString(e), grid, threads, lds);
    return SPECQ_EIO;
  }
  return SPECQ_OK;
}

int ensure_lds(const void* fn, size_t lds) {
  if (lds <= 65536) return SPECQ_OK;
  static std::mutex mu;
  static std::set<const void*> done;
  std::lock_guard<std::mutex> lock(mu);
  if (done.count(fn)) return SPECQ_OK;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) {
    set_error("cannot enable %zu bytes of LDS: %s", lds, hipGetErrorString(e));
    return SPECQ_EIO;
  }
  done.insert(fn);
  return SPECQ_OK;
}

int device_cus() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cache[dev] = cus;
  }
  return cache[dev];
}

int w8a8_attrs(int layout, int m_grid, int N, int K, int block_m, int block_n, int num_warps, int split_k,
               specq_kernel_attrs* out);
int w4a16_attrs(int layout, int m_grid, int N, int K, int block_m, int block_n, int num_warps, int split_k,
                specq_kernel_attrs* out);
int attn_attrs(int D, int rows, specq_kernel_attrs* out);

}  // namespace specq

extern "C" int specq_version(void) { return 100; }

extern "C" const char* specq_last_error(void) { return specq::g_err; }

extern "C" int specq_kernel_attrs_query(int kind, int variant, int m_grid, int N, int K, int block_m, int block_n,
                                        int num_warps, int split_k, specq_kernel_attrs* out) {
  specq::clear_error();
  if (!out) return specq::fail(SPECQ_EINVAL, "kernel_attrs: null output");
  memset(out, 0, sizeof(*out));
  switch (kind) {
    case 0: return specq::w8a8_attrs(variant, m_grid, N, K, block_m, block_n, num_warps, split_k, out);
    case 1: return specq::w4a16_attrs(variant, m_grid, N, K, block_m, block_n, num_warps, split_k, out);
    case 2: return specq::attn_attrs(variant, block_m, out);
  }
  return specq::fail(SPECQ_EINVAL, "kernel_attrs: unknown kind");
}
