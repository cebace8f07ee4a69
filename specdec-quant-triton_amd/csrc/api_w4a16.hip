// C ABI for the W4A16 GEMM: argument validation, tile / split-K selection and launch.
#include "api_common.hpp"
#include "w4a16.hpp"

namespace specq {

const void* w4a16_kernel_l0(int mt, int rw);
const void* w4a16_kernel_l1(int mt, int rw);

namespace {

constexpr int kW4Waves = 4;

struct W4Cfg {
  int mt, rw, splits, bps, n_tiles, m_chunks, nblocks;
  size_t lds, ws_partials, ws_counters;
  const void* fn;
};

int w4_config(int layout, int m_grid, int N, int K, int block_m, int block_n, int split_k, W4Cfg* cfg) {
  SPECQ_REQUIRE(layout == 0 || layout == 1, SPECQ_EINVAL, "w4a16: unknown weight layout %d", layout);
  SPECQ_REQUIRE(m_grid >= 0 && N > 0 && K > 0, SPECQ_EINVAL, "w4a16: bad sizes M=%d N=%d K=%d", m_grid, N, K);
  SPECQ_REQUIRE(K % 128 == 0, SPECQ_ENOTSUP, "w4a16: K=%d must be a multiple of 128", K);
  const int rows16 = ceil_div(m_grid > 0 ? m_grid : 1, 16);
  int mt;
  if (block_m > 0) {
    SPECQ_REQUIRE(block_m % 16 == 0 && block_m <= 256, SPECQ_ENOTSUP,
                  "w4a16: BLOCK_M=%d must be a multiple of 16 and at most 256", block_m);
    mt = block_m / 16;
  } else {
    // Wide N: one M-chunk up to 256 rows (one weight pass); narrow N: 48-row chunks, so more
    // workgroups share the activation traffic (measured on the Llama-3-8B linears).
    const int cap = ceil_div(N, 64) >= 128 ? 16 : 3;
    const int chunks = ceil_div(rows16, cap);
    mt = ceil_div(rows16, chunks);
  }
  // BLOCK_N is the channel width of the whole workgroup (4 waves): 64 or 128.
  int rw = 1;
  if (block_n > 0) {
    SPECQ_REQUIRE(block_n == 64 || block_n == 128, SPECQ_ENOTSUP, "w4a16: BLOCK_N=%d must be 64 or 128", block_n);
    rw = block_n / 64;
  }
  cfg->mt = mt; cfg->rw = rw;
  cfg->n_tiles = ceil_div(N, kW4Waves * rw * 16);
  cfg->m_chunks = ceil_div(m_grid > 0 ? m_grid : 1, mt * 16);
  cfg->nblocks = K / 128;
  int splits;
  if (split_k > 0) {
    splits = split_k;
  } else {
    // A function of (N, K, BLOCK_N) only, so the fp32 summation order never depends on M:
    // about two workgroups per CU, each split long enough (>= 8 blocks) to fill its prefetch ring.
    const int target = 2 * device_cus();
    splits = cfg->n_tiles >= target ? 1 : ceil_div(target, cfg->n_tiles);
    int max_splits = cfg->nblocks / 8;
    if (max_splits < 1) max_splits = 1;
    if (splits > max_splits) splits = max_splits;
  }
  if (splits > cfg->nblocks) splits = cfg->nblocks;
  cfg->bps = ceil_div(cfg->nblocks, splits);
  cfg->splits = ceil_div(cfg->nblocks, cfg->bps);
  const int BM = mt * 16, BN = kW4Waves * rw * 16;
  cfg->lds = 0;  // static LDS (activation ring slots)
  cfg->ws_partials = cfg->splits > 1 ? align_up((size_t)cfg->m_chunks * cfg->n_tiles * cfg->splits * BM * BN * 4, 256) : 0;
  cfg->ws_counters = cfg->splits > 1 ? kCounterBytes : 0;
  SPECQ_REQUIRE((int64_t)cfg->m_chunks * cfg->n_tiles <= kMaxCounters, SPECQ_ENOTSUP,
                "w4a16: %d x %d tiles exceed the counter region", cfg->m_chunks, cfg->n_tiles);
  cfg->fn = layout == 0 ? w4a16_kernel_l0(mt, rw) : w4a16_kernel_l1(mt, rw);
  SPECQ_REQUIRE(cfg->fn != nullptr, SPECQ_ENOTSUP, "w4a16: kernel MT=%d RW=%d not built", mt, rw);
  return SPECQ_OK;
}

}  // namespace

int w4a16_attrs(int layout, int m_grid, int N, int K, int block_m, int block_n, int num_warps, int split_k,
                specq_kernel_attrs* out) {
  (void)num_warps;
  W4Cfg cfg;
  int rc = w4_config(layout, m_grid, N, K, block_m, block_n, split_k, &cfg);
  if (rc) return rc;
  hipFuncAttributes fa;
  if (hipFuncGetAttributes(&fa, cfg.fn) != hipSuccess) return fail(SPECQ_EIO, "w4a16: hipFuncGetAttributes failed");
  snprintf(out->name, sizeof(out->name), "specq::w4a16_kernel<%d,%d,%d>", cfg.mt, cfg.rw, layout);
  out->num_regs = fa.numRegs;
  out->lds_bytes = (int)(fa.sharedSizeBytes + cfg.lds);
  out->scratch_bytes = (int)fa.localSizeBytes;
  out->threads = kW4Waves * 64;
  out->grid = cfg.m_chunks * cfg.n_tiles * cfg.splits;
  out->block_m = cfg.mt * 16; out->block_n = kW4Waves * cfg.rw * 16; out->num_warps = kW4Waves;
  out->split_k = cfg.splits;
  return SPECQ_OK;
}

}  // namespace specq

using namespace specq;

extern "C" size_t specq_w4a16_workspace_size(int m_grid, int N, int K, int block_m, int block_n, int num_warps,
                                             int split_k) {
  (void)num_warps;
  W4Cfg cfg;
  size_t need = 0;
  if (w4_config(1, m_grid, N, K, block_m, block_n, split_k, &cfg) == SPECQ_OK) need = cfg.ws_partials + cfg.ws_counters;
  clear_error();
  return need;
}

extern "C" int specq_w4a16(const void* a, int64_t lda, const void* wq, int64_t ldq, int wq_layout, const void* sc,
                           int64_t ld_sc, void* c, int64_t ldc, int M, int N, int K, int group, int grid_m_max,
                           const int32_t* plan, int block_m, int block_n, int num_warps, int split_k, void* workspace,
                           size_t workspace_bytes, void* stream) {
  (void)num_warps;
  clear_error();
  SPECQ_REQUIRE(M >= 0 && N > 0 && K > 0, SPECQ_EINVAL, "w4a16: bad sizes M=%d N=%d K=%d", M, N, K);
  SPECQ_REQUIRE(a && wq && sc && c, SPECQ_EINVAL, "w4a16: null tensor pointer");
  SPECQ_REQUIRE(wq_layout == 0 || wq_layout == 1, SPECQ_EINVAL, "w4a16: unknown weight layout %d", wq_layout);
  SPECQ_REQUIRE(group > 0 && K % group == 0, SPECQ_EINVAL, "w4a16: group=%d must divide K=%d", group, K);
  SPECQ_REQUIRE(group % (wq_layout == 1 ? 32 : 16) == 0 && (group & (group - 1)) == 0, SPECQ_ENOTSUP,
                "w4a16: group=%d must be a power of two and a multiple of %d for layout %d", group,
                wq_layout == 1 ? 32 : 16, wq_layout);
  const int64_t row_bytes = wq_layout == 1 ? ldq * 4 : ldq;
  SPECQ_REQUIRE(lda >= K && row_bytes >= K / 2 && ld_sc >= K / group && ldc >= N, SPECQ_EINVAL,
                "w4a16: row strides must cover a row");
  SPECQ_REQUIRE(grid_m_max == 0 || grid_m_max >= M, SPECQ_EINVAL, "w4a16: grid_m_max=%d < M=%d", grid_m_max, M);
  SPECQ_REQUIRE((uintptr_t)a % 16 == 0 && lda % 8 == 0, SPECQ_ENOTSUP,
                "w4a16: activations need 16-byte aligned rows (lda %% 8 == 0)");
  SPECQ_REQUIRE((uintptr_t)wq % 16 == 0 && row_bytes % 16 == 0, SPECQ_ENOTSUP,
                "w4a16: packed weights need 16-byte aligned rows");
  SPECQ_REQUIRE((uintptr_t)sc % 2 == 0, SPECQ_EINVAL, "w4a16: misaligned scales");
  const int m_grid = grid_m_max > 0 ? grid_m_max : M;
  if (m_grid == 0) return SPECQ_OK;
  W4Cfg cfg;
  int rc = w4_config(wq_layout, m_grid, N, K, block_m, block_n, split_k, &cfg);
  if (rc) return rc;
  const size_t need = cfg.ws_partials + cfg.ws_counters;
  SPECQ_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), SPECQ_ENOSPC,
                "w4a16: workspace of %zu bytes required, %zu given", need, workspace ? workspace_bytes : 0);
  rc = ensure_lds(cfg.fn, cfg.lds);
  if (rc) return rc;
  W4A16Params p;
  p.A = (const _Float16*)a; p.lda = lda; p.Wq = (const uint8_t*)wq; p.ldq = row_bytes;
  p.sc = (const _Float16*)sc; p.ld_sc = ld_sc; p.C = (_Float16*)c; p.ldc = ldc; p.plan = plan;
  p.M = M; p.N = N; p.K = K; p.group = group; p.m_grid = m_grid;
  p.group_shift = __builtin_ctz((unsigned)group);
  p.n_tiles = cfg.n_tiles; p.m_chunks = cfg.m_chunks; p.splits = cfg.splits; p.nblocks = cfg.nblocks;
  p.blocks_per_split = cfg.bps;
  p.counters = need ? (int32_t*)workspace : nullptr;
  p.partials = need ? (float*)((char*)workspace + kCounterBytes) : nullptr;
  p.vec_store = ((uintptr_t)c % 8 == 0) && (ldc % 4 == 0);
  const int grid = cfg.m_chunks * cfg.n_tiles * cfg.splits;
  return launch(cfg.fn, grid, kW4Waves * 64, cfg.lds, (hipStream_t)stream, &p);
}
