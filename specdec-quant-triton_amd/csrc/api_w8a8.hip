// C ABI for the W8A8 GEMM: argument validation, tile / split-K selection and launch.
#include "api_common.hpp"
#include "w8a8.hpp"

namespace specq {

const void* w8a8_kernel_rw1(int mt, int vec);
const void* w8a8_kernel_rw2(int mt, int vec);
const void* w8a8_kernel_rw4(int mt, int vec);

namespace {

struct W8A8Cfg {
  int mt, rw, nw, vec, splits, k_range, n_tiles, m_chunks;
  size_t lds, ws_partials, ws_counters;
  const void* fn;
};

// MT values built for operands that are not 16-byte aligned.
int round_mt_for_vec(int mt, int vec, int rw) {
  if (vec == 16) return mt;
  static const int avail[] = {1, 2, 4, 8, 16, 20};
  for (int a : avail)
    if (a >= mt && a * rw <= 40) return a;
  return -1;
}

const void* w8a8_fn(int mt, int rw, int vec) {
  switch (rw) {
    case 1: return w8a8_kernel_rw1(mt, vec);
    case 2: return w8a8_kernel_rw2(mt, vec);
    case 4: return w8a8_kernel_rw4(mt, vec);
  }
  return nullptr;
}

// Resolve the tile configuration.  `vec` is the operand alignment (16 when unknown).
int w8a8_config(int m_grid, int N, int K, int block_m, int block_n, int num_warps, int split_k, int vec,
                W8A8Cfg* cfg) {
  SPECQ_REQUIRE(m_grid >= 0 && N > 0 && K > 0, SPECQ_EINVAL, "w8a8: bad sizes M=%d N=%d K=%d", m_grid, N, K);
  int rows16 = ceil_div(m_grid > 0 ? m_grid : 1, 16);
  int mt;
  if (block_m > 0) {
    SPECQ_REQUIRE(block_m % 16 == 0 && block_m <= 320, SPECQ_ENOTSUP,
                  "w8a8: BLOCK_M=%d must be a multiple of 16 and at most 320", block_m);
    mt = block_m / 16;
  } else {
    int chunks = ceil_div(rows16, 20);
    mt = ceil_div(rows16, chunks);
  }
  int rw;
  if (block_n > 0) {
    SPECQ_REQUIRE(block_n == 16 || block_n == 32 || block_n == 64, SPECQ_ENOTSUP,
                  "w8a8: BLOCK_N=%d must be 16, 32 or 64", block_n);
    rw = block_n / 16;
  } else {
    rw = N <= 16 ? 1 : 2;
  }
  while (rw > 1 && rw * mt > 40) rw >>= 1;
  int mt_eff = round_mt_for_vec(mt, vec, rw);
  if (mt_eff < 0 && rw > 1) { rw = 1; mt_eff = round_mt_for_vec(mt, vec, rw); }
  SPECQ_REQUIRE(mt_eff > 0, SPECQ_ENOTSUP, "w8a8: no kernel for BLOCK_M=%d at %d-byte alignment", mt * 16, vec);
  mt = mt_eff;
  int nw = num_warps <= 0 ? 4 : (num_warps >= 4 ? 4 : (num_warps >= 2 ? 2 : 1));

  cfg->mt = mt; cfg->rw = rw; cfg->nw = nw; cfg->vec = vec;
  cfg->n_tiles = ceil_div(N, rw * 16);
  cfg->m_chunks = ceil_div(m_grid > 0 ? m_grid : 1, mt * 16);
  const int ksteps = ceil_div(K, 64);
  int splits;
  if (split_k > 0) {
    splits = split_k;
  } else {
    // Aim for about two resident workgroups per CU, and keep at least 2 K steps per wave.
    const int target = 2 * device_cus();
    const int base = cfg->n_tiles * cfg->m_chunks;
    splits = base >= target ? 1 : ceil_div(target, base);
    int max_splits = ksteps / (2 * nw);
    if (max_splits < 1) max_splits = 1;
    if (splits > max_splits) splits = max_splits;
  }
  if (splits > ksteps) splits = ksteps;
  int k_range = ceil_div(ksteps, splits) * 64;
  splits = ceil_div(K, k_range);
  cfg->splits = splits;
  cfg->k_range = k_range;
  const int BM = mt * 16, BN = rw * 16;
  cfg->lds = nw > 1 ? (size_t)BM * (BN + kW8A8Pad) * 4 : 0;
  cfg->ws_partials = splits > 1 ? align_up((size_t)cfg->m_chunks * cfg->n_tiles * splits * BM * BN * 4, 256) : 0;
  cfg->ws_counters = splits > 1 ? kCounterBytes : 0;
  SPECQ_REQUIRE((int64_t)cfg->m_chunks * cfg->n_tiles <= kMaxCounters, SPECQ_ENOTSUP,
                "w8a8: %d x %d tiles exceed the counter region", cfg->m_chunks, cfg->n_tiles);
  cfg->fn = w8a8_fn(mt, rw, vec);
  SPECQ_REQUIRE(cfg->fn != nullptr, SPECQ_ENOTSUP, "w8a8: kernel MT=%d RW=%d VEC=%d not built", mt, rw, vec);
  return SPECQ_OK;
}

}  // namespace

int w8a8_attrs(int m_grid, int N, int K, int block_m, int block_n, int num_warps, int split_k,
               specq_kernel_attrs* out) {
  W8A8Cfg cfg;
  int rc = w8a8_config(m_grid, N, K, block_m, block_n, num_warps, split_k, 16, &cfg);
  if (rc) return rc;
  hipFuncAttributes fa;
  if (hipFuncGetAttributes(&fa, cfg.fn) != hipSuccess) return fail(SPECQ_EIO, "w8a8: hipFuncGetAttributes failed");
  snprintf(out->name, sizeof(out->name), "specq::w8a8_kernel<%d,%d,%d>", cfg.mt, cfg.rw, cfg.vec);
  out->num_regs = fa.numRegs;
  out->lds_bytes = (int)(fa.sharedSizeBytes + cfg.lds);
  out->scratch_bytes = (int)fa.localSizeBytes;
  out->threads = cfg.nw * 64;
  out->grid = cfg.m_chunks * cfg.n_tiles * cfg.splits;
  out->block_m = cfg.mt * 16; out->block_n = cfg.rw * 16; out->num_warps = cfg.nw; out->split_k = cfg.splits;
  return SPECQ_OK;
}

}  // namespace specq

using namespace specq;

extern "C" size_t specq_w8a8_workspace_size(int m_grid, int N, int K, int block_m, int block_n, int num_warps,
                                            int split_k) {
  W8A8Cfg cfg;
  // Sub-16-byte alignments only ever round MT up, which can only shrink the split count's
  // base; size for the worst case over the alignments.
  size_t best = 0;
  for (int vec : {16, 1}) {
    if (w8a8_config(m_grid, N, K, block_m, block_n, num_warps, split_k, vec, &cfg) == SPECQ_OK) {
      size_t s = cfg.ws_partials + cfg.ws_counters;
      if (s > best) best = s;
    }
  }
  clear_error();
  return best;
}

extern "C" int specq_w8a8(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, const float* sa,
                          const float* sw, void* c, int64_t ldc, int M, int N, int K, int grid_m_max,
                          const int32_t* plan, int block_m, int block_n, int num_warps, int split_k,
                          void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  SPECQ_REQUIRE(M >= 0 && N > 0 && K > 0, SPECQ_EINVAL, "w8a8: bad sizes M=%d N=%d K=%d", M, N, K);
  SPECQ_REQUIRE(a && w && sa && sw && c, SPECQ_EINVAL, "w8a8: null tensor pointer");
  SPECQ_REQUIRE(lda >= K && ldw >= K && ldc >= N, SPECQ_EINVAL,
                "w8a8: row strides must cover a row (lda=%lld ldw=%lld ldc=%lld)", (long long)lda,
                (long long)ldw, (long long)ldc);
  SPECQ_REQUIRE(grid_m_max == 0 || grid_m_max >= M, SPECQ_EINVAL, "w8a8: grid_m_max=%d < M=%d", grid_m_max, M);
  const int m_grid = grid_m_max > 0 ? grid_m_max : M;
  if (m_grid == 0) return SPECQ_OK;
  const int vec = common_vec({(uint64_t)(uintptr_t)a, (uint64_t)(uintptr_t)w, (uint64_t)lda, (uint64_t)ldw,
                              (uint64_t)K});
  W8A8Cfg cfg;
  int rc = w8a8_config(m_grid, N, K, block_m, block_n, num_warps, split_k, vec, &cfg);
  if (rc) return rc;
  const size_t need = cfg.ws_partials + cfg.ws_counters;
  SPECQ_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), SPECQ_ENOSPC,
                "w8a8: workspace of %zu bytes required, %zu given", need, workspace ? workspace_bytes : 0);
  W8A8Params p;
  p.A = a; p.lda = lda; p.W = w; p.ldw = ldw; p.sa = sa; p.sw = sw;
  p.C = reinterpret_cast<__half*>(c); p.ldc = ldc; p.plan = plan;
  p.M = M; p.N = N; p.K = K; p.m_grid = m_grid;
  p.n_tiles = cfg.n_tiles; p.m_chunks = cfg.m_chunks; p.splits = cfg.splits; p.k_range = cfg.k_range;
  p.counters = need ? reinterpret_cast<int32_t*>(workspace) : nullptr;
  p.partials = need ? reinterpret_cast<int32_t*>(reinterpret_cast<char*>(workspace) + kCounterBytes) : nullptr;
  p.vec_store = ((uintptr_t)c % 8 == 0) && (ldc % 4 == 0) && ((uintptr_t)sw % 16 == 0);
  const int grid = cfg.m_chunks * cfg.n_tiles * cfg.splits;
  return launch(cfg.fn, grid, cfg.nw * 64, cfg.lds, reinterpret_cast<hipStream_t>(stream), &p);
}
