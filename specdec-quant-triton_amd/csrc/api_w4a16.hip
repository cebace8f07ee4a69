// C ABI for the W4A16 GEMM: argument validation, split / tile / kernel-family selection,
// launch, and the load-time weight packing.
//
// Kernel families (identical fp32 summation order, so every choice is bit-identical):
//   WS  LDS-staged activations (w4a16_ws.hpp) for token tiles up to 160 rows (default; a
//       deeper BLOCK_M runs as equal chunks of at most 160 rows).
//   RK  register-stream kernel (w4a16_rk.hpp) for 16- and 32-row token tiles (w4a16_path 1).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <map>
#include <mutex>

#include "api_common.hpp"
#include "w4a16_plan.hpp"
#include "w4a16_tiles.hpp"

namespace specq {

const void* w4a16_plan_fn_l0();  // w4a16_plan_l*.hip
const void* w4a16_plan_fn_l1();
const void* w4a16_plan_fn_l2();

// Packs a W4A16 weight (layout 0 or 1, row stride ldq bytes) into 1 KB MFMA fragments:
// fragment (b, t) of K block b and 16-row tile t at (b * ntiles + t) KB; lane l's 16 bytes hold
// the nibbles of row 16t + l%16 for k = 128b + 32*(l/16) + 8u + j as word u, nibble j at bits
// 4p..4p+3 with p = j/2 for even j and 4 + j/2 for odd j.  Rows past N hold nibble 8 (weight 0).
__global__ __launch_bounds__(256) void w4a16_pack_kernel(const uint8_t* __restrict__ wq, int64_t ldq, int layout,
                                                         int N, int K, uint8_t* __restrict__ out) {
  const int ntiles = (N + 15) / 16;
  const int nblocks = K / 128;
  const int64_t frag = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // one wave per fragment
  if (frag >= (int64_t)ntiles * nblocks) return;
  const int b = (int)(frag / ntiles), t = (int)(frag % ntiles);
  const int l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const int row = 16 * t + r;
  const uint8_t* src = wq + (int64_t)min(row, N - 1) * ldq;
  auto nib = [&](int k) -> uint32_t {
    if (row >= N) return 8u;
    if (layout == 0) {
      const int half = K / 2;
      return k < half ? (src[k] & 15u) : (src[k - half] >> 4);
    }
    return (src[k >> 1] >> (4 * (k & 1))) & 15u;  // int32 words in k order = bytes in k order
  };
  // Weight j of a word at nibble position (j odd ? 4 : 0) + j / 2 (w4_dequant_packed).
  int words[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int k0 = 128 * b + 32 * g + 8 * u;
    uint32_t x = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) x |= nib(k0 + j) << (4 * ((j & 1) * 4 + (j >> 1)));
    words[u] = (int)x;
  }
  *reinterpret_cast<v4i*>(out + frag * 1024 + l * 16) = v4i{words[0], words[1], words[2], words[3]};
}

// Kernel family override (0 = automatic), set through specq_set_option("w4a16_path", v).
std::atomic<int> g_w4a16_path{0};

namespace {

// kW4Plan: plan-mode launch holding the menu of LDS-staged tilings (w4a16_plan.hpp), one per
// 16 rows of the active M.
enum W4Family { kW4Rk = 1, kW4Ws = 2, kW4Plan = 3 };

struct W4Cfg {
  int family, layout, mt, rw, splits, bps, n_tiles, m_chunks, units, grid, nblocks;
  size_t ws_partials, ws_counters;
  const void* fn;
  W4PlanTile plan_t[kW4PlanRows];  // kW4Plan: the tiling of each 16-row step of M
};

// Split count: a function of (N, K) only (or the caller's split_k), so the fp32 summation
// order never depends on M, the token tile or the plan.  Wide N already fills the CUs with
// 64-channel tiles; narrower N is split along K into about 256 workgroups, each at least 4
// blocks (512 K) long.
// Split count of the K range, a function of (N, K) only so that the fp32 summation order (and
// with it every result) is the same for every M, tile and plan mode.  Measured on the
// Llama-3-8B linears (qkv, o, gate_up, down, gate, k/v at M = 8..288): the most splits, a
// power of two, that keep the 64-channel tiles x splits within one workgroup per CU and at
// least 8 K blocks (1024 of K) per split; two rounds of workgroups or shorter splits lose.
int w4_auto_splits(int N, int nblocks) {
  const int tiles64 = ceil_div(N, 64);
  const int cus = device_cus();
  int splits = 1;
  while (tiles64 * splits * 2 <= cus && nblocks / (splits * 2) >= 8) splits *= 2;
  return splits;
}

// Eager tile choice for M > 16 over the token-tile depth (M cut into c = 1..6 chunks) and the
// channel block (64 or 128), from a model fitted to 130 measured shapes x tiles of the
// Llama-3-8B linears at M = 8..288 (mean regret 4.5 % against the best measured tile; one chunk
// over all of M lost 21 % on average and up to 2.7x at M >= 192).  Per workgroup round:
//   max(activation + weight intake at 60 GB/s per CU, dequant and MFMA work), against all
//   weights at 7 TB/s, plus 2 us.
// The split count is the caller's or w4_auto_splits(N, K), so the summation order, and with it
// every result, is the same for every tile.
// Modelled time of one tiling (token-tile depth mt, rw 64-channel fragments) of `rows16` token
// tiles with `splits` K splits on `cus` CUs, from the model above.
double w4_model_time(int rows16, int N, int K, int splits, int mt, int rw, int cus) {
  const int chunks = ceil_div(rows16, mt), rows = mt * 16;
  const int bn = 64 * rw;
  const double rounds = (double)ceil_div(ceil_div(N, bn) * splits * chunks, cus);
  const double kk = (double)K / splits;
  const double t_in = rounds * (bn * 0.5 + rows * 2.0) * kk / 60e3;
  const double t_work = rounds * (bn * kk * 8e-6 + (double)rows * bn * kk * 4e-7);
  return std::max(std::max(t_in, t_work), (double)N * K * 0.5 / 7e6) + 2.0;
}

void w4_auto_tiles(int M, int N, int K, int splits, int rw_fixed, int* mt_out, int* rw_out) {
  const int cus = device_cus();
  const int rows16 = ceil_div(std::max(M, 1), 16);
  double best_t = 0;
  int best_mt = -1, best_rw = 1, last_mt = -1;
  // At most the deepest compiled tile (160 rows), so M up to 320 runs as at most two chunks.
  constexpr int kMaxAutoMt = kW4MaxMt;
  const int max_c = std::max(6, ceil_div(rows16, kMaxAutoMt));
  for (int c = 1; c <= max_c; ++c) {
    const int mt = ceil_div(rows16, c);
    if (mt == last_mt || mt > kMaxAutoMt) continue;
    last_mt = mt;
    for (int rw = 1; rw <= 2; ++rw) {
      if (rw_fixed > 0 && rw != rw_fixed) continue;
      const double t = w4_model_time(rows16, N, K, splits, mt, rw, cus);
      if (best_mt < 0 || t < best_t) { best_t = t; best_mt = mt; best_rw = rw; }
    }
  }
  *mt_out = best_mt;
  *rw_out = best_rw;
}

// Plan-mode calls with automatic tiles: the per-16-row table of w4a16_plan_kernel, each step's
// menu tiling priced lowest by the eager model at the step's largest M (the decode rule at
// M <= 16), every entry with the split count of (N, K).  Equal prices go to fewer workgroups,
// then to the shallower tile.  Tables are cached per shape.
int w4_plan_config(int layout, int m_grid, int N, int K, int split_k, W4Cfg* cfg) {
  const int cus = device_cus();
  struct Key {
    int v[6];
    bool operator<(const Key& o) const { return std::lexicographical_compare(v, v + 6, o.v, o.v + 6); }
  };
  const Key key{{cus, layout, m_grid, N, K, split_k}};
  static std::mutex mu;
  static std::map<Key, W4Cfg> cache;
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) {
      *cfg = it->second;
      return SPECQ_OK;
    }
  }
  const int R = ceil_div(std::max(m_grid, 1), 16);
  cfg->family = kW4Plan; cfg->layout = layout;
  cfg->nblocks = K / 128;
  int splits = split_k > 0 ? split_k : w4_auto_splits(N, cfg->nblocks);
  if (splits > cfg->nblocks) splits = cfg->nblocks;
  cfg->bps = ceil_div(cfg->nblocks, splits);
  cfg->splits = ceil_div(cfg->nblocks, cfg->bps);
  size_t ws = 0;
  int grid = 0;
  for (int e = 0; e < kW4PlanRows; ++e) {
    const int r = e == kW4PlanRows - 1 ? R : std::min(e + 1, R);
    int path = -1;
    if (r == 1) {
      path = ceil_div(N, 64) > cus ? 1 : 0;  // 16-row tile; 128 channels keep wide N to one round
    } else {
      double best = 0;
      int64_t best_wgs = 0;
      for (int i = 0; i < kW4PlanMenu; ++i) {
        const int mt = kW4PlanMenuMt[i], rw = kW4PlanMenuRw[i];
        const double t = w4_model_time(r, N, K, cfg->splits, mt, rw, cus);
        const int64_t wgs = (int64_t)ceil_div(N, 64 * rw) * cfg->splits * ceil_div(r, mt);
        const bool tie = path >= 0 && std::fabs(t - best) <= 1e-9 * best;
        if (path < 0 || (t < best && !tie) ||
            (tie && (wgs < best_wgs || (wgs == best_wgs && mt < kW4PlanMenuMt[path])))) {
          best = t; path = i; best_wgs = wgs;
        }
      }
    }
    const int mt = kW4PlanMenuMt[path], rw = kW4PlanMenuRw[path];
    W4PlanTile& t = cfg->plan_t[e];
    t.path = path;
    t.n_tiles = ceil_div(N, 64 * rw);
    t.m_chunks = ceil_div(r, mt);
    SPECQ_REQUIRE((int64_t)t.m_chunks * t.n_tiles <= kMaxCounters, SPECQ_ENOTSUP,
                  "w4a16 plan: %d x %d tiles exceed the counter region", t.m_chunks, t.n_tiles);
    if (cfg->splits > 1)
      ws = std::max(ws, align_up((size_t)t.m_chunks * t.n_tiles * cfg->splits * (mt * 16) * (64 * rw) * 4, 256));
    grid = std::max(grid, chunked_grid(t.n_tiles * cfg->splits, t.m_chunks));
  }
  const W4PlanTile& top = cfg->plan_t[std::min(R, kW4PlanRows) - 1];
  cfg->mt = kW4PlanMenuMt[top.path];
  cfg->rw = kW4PlanMenuRw[top.path];
  cfg->n_tiles = top.n_tiles;
  cfg->m_chunks = top.m_chunks;
  cfg->units = cfg->n_tiles * cfg->splits;
  cfg->grid = grid;
  cfg->ws_partials = ws;
  cfg->ws_counters = cfg->splits > 1 ? kCounterBytes : 0;
  cfg->fn = layout == 0 ? w4a16_plan_fn_l0() : (layout == 1 ? w4a16_plan_fn_l1() : w4a16_plan_fn_l2());
  std::lock_guard<std::mutex> lock(mu);
  cache[key] = *cfg;
  return SPECQ_OK;
}

int w4_config(int layout, int m_grid, int N, int K, int block_m, int block_n, int split_k, bool plan_mode,
              W4Cfg* cfg, bool allow_menu = true) {
  SPECQ_REQUIRE(layout >= 0 && layout <= 2, SPECQ_EINVAL, "w4a16: unknown weight layout %d", layout);
  SPECQ_REQUIRE(m_grid >= 0 && N > 0 && K > 0, SPECQ_EINVAL, "w4a16: bad sizes M=%d N=%d K=%d", m_grid, N, K);
  SPECQ_REQUIRE(K % 128 == 0, SPECQ_ENOTSUP, "w4a16: K=%d must be a multiple of 128", K);
  const int rows16 = ceil_div(m_grid > 0 ? m_grid : 1, 16);
  if (allow_menu && plan_mode && block_m <= 0 && block_n <= 0 && g_w4a16_path.load() == 0)
    return w4_plan_config(layout, m_grid, N, K, split_k, cfg);
  int mt;
  if (block_m > 0) {
    SPECQ_REQUIRE(block_m % 16 == 0 && block_m <= 256, SPECQ_ENOTSUP,
                  "w4a16: BLOCK_M=%d must be a multiple of 16 and at most 256", block_m);
    // Tiles deeper than the deepest compiled one run as equal chunks of at most that depth
    // (the result does not depend on the tiling).
    const int req = block_m / 16;
    mt = ceil_div(req, ceil_div(req, kW4MaxMt));
  } else {
    // One chunk of token rows covering M (the weight is read once), split evenly past the
    // deepest tile.  With a plan the active M is usually far below the grid's: chunks of at
    // most 80 rows let the chunks past the active M exit at once.
    const int cap = plan_mode ? 5 : kW4MaxMt;
    const int chunks = ceil_div(rows16, cap);
    mt = ceil_div(rows16, chunks);
  }
  int rw = 1;
  if (block_n > 0) {
    SPECQ_REQUIRE(block_n == 64 || block_n == 128, SPECQ_ENOTSUP, "w4a16: BLOCK_N=%d must be 64 or 128", block_n);
    rw = block_n / 64;
  } else if (ceil_div(N, 64) > device_cus()) {
    rw = 2;  // 128-channel blocks keep wide N (the fused gate_up) to one workgroup per CU
  }
  int t_bm = 0, t_bn = 0, t_sk = 0;
  if (block_m <= 0 && block_n <= 0 && !plan_mode && tuned_tile(1, N, K, std::max(m_grid, 1), &t_bm, &t_bn, &t_sk)) {
    // A launch shape of the measured table: its tile (the split count still follows N and K).
    mt = t_bm / 16;
    rw = t_bn / 64;
  } else if (block_m <= 0 && !plan_mode && rows16 > 1) {
    const int nb = K / 128;
    const int s_auto = std::min(split_k > 0 ? split_k : w4_auto_splits(N, nb), nb);
    const int s_eff = ceil_div(nb, ceil_div(nb, s_auto));
    w4_auto_tiles(m_grid, N, K, s_eff, block_n > 0 ? rw : 0, &mt, &rw);
  }
  // The LDS-staged kernel is the default at every depth (measured faster than the register
  // stream even for 16-row tiles on the Llama-3-8B linears); the register stream stays
  // selectable for tiles of up to 32 rows.
  const int path = g_w4a16_path.load();
  const int family = (path == kW4Rk && mt <= kW4RkMaxMt) ? kW4Rk : kW4Ws;

  cfg->family = family; cfg->layout = layout; cfg->mt = mt; cfg->rw = rw;
  cfg->nblocks = K / 128;
  cfg->n_tiles = ceil_div(N, 64 * rw);
  cfg->m_chunks = ceil_div(m_grid > 0 ? m_grid : 1, mt * 16);
  int splits = split_k > 0 ? split_k : w4_auto_splits(N, cfg->nblocks);
  if (splits > cfg->nblocks) splits = cfg->nblocks;
  cfg->bps = ceil_div(cfg->nblocks, splits);
  cfg->splits = ceil_div(cfg->nblocks, cfg->bps);
  cfg->units = cfg->n_tiles * cfg->splits;
  cfg->grid = chunked_grid(cfg->units, cfg->m_chunks);
  const int BM = mt * 16, BN = 64 * rw;
  cfg->ws_partials = cfg->splits > 1 ? align_up((size_t)cfg->m_chunks * cfg->n_tiles * cfg->splits * BM * BN * 4, 256) : 0;
  cfg->ws_counters = cfg->splits > 1 ? kCounterBytes : 0;
  SPECQ_REQUIRE((int64_t)cfg->m_chunks * cfg->n_tiles <= kMaxCounters, SPECQ_ENOTSUP,
                "w4a16: %d x %d tiles exceed the counter region", cfg->m_chunks, cfg->n_tiles);
  if (family == kW4Rk) {
    cfg->fn = w4a16_rk_fn(mt, rw, layout);
  } else {
    switch (layout) {
      case 0: cfg->fn = w4a16_ws_fn_l0(mt, rw); break;
      case 1: cfg->fn = w4a16_ws_fn_l1(mt, rw); break;
      default: cfg->fn = w4a16_ws_fn_l2(mt, rw); break;
    }
  }
  SPECQ_REQUIRE(cfg->fn != nullptr, SPECQ_ENOTSUP, "w4a16: no kernel for BLOCK_M=%d BLOCK_N=%d", mt * 16, 64 * rw);
  return SPECQ_OK;
}

size_t w4_workspace(int m_grid, int N, int K, int block_m, int block_n, int split_k) {
  // The partial-tile region does not depend on the weight layout or kernel family; take the
  // larger of the eager and plan-mode token tilings.
  size_t need = 0;
  for (int plan_mode = 0; plan_mode < 2; ++plan_mode) {
    W4Cfg cfg;
    if (w4_config(1, m_grid, N, K, block_m, block_n, split_k, plan_mode != 0, &cfg) == SPECQ_OK) {
      const size_t n = cfg.ws_partials + cfg.ws_counters;
      need = n > need ? n : need;
    }
  }
  clear_error();
  return need;
}

// Split count of every member of a grouped launch (the caller's, or each member's own
// w4_auto_splits, which must then agree), so each member sums K exactly as its own call would.
// 0 when the members' automatic counts differ.
int w4_group_splits(int n_members, const int* N, int K, int split_k) {
  const int nb = K / 128;
  int common = -1;
  for (int g = 0; g < n_members; ++g) {
    int s = split_k > 0 ? split_k : w4_auto_splits(N[g], nb);
    if (s > nb) s = nb;
    s = ceil_div(nb, ceil_div(nb, s));  // the count a call with this request runs
    if (common >= 0 && s != common) return 0;
    common = s;
  }
  return common;
}

// Tiles of a grouped launch: chosen as for one GEMM of the members' total width (never the
// plan-mode menu: a plan-mode grouped call runs the streaming kernel at the tiles of its grid's
// M, reading the active M on the device), every member with the common split count; each
// member's channel tiles start a new tile, so the launch-wide tile count is the members' sum.
int w4_group_config(int layout, int m_grid, int n_members, const int* N, int K, int block_m, int block_n,
                    int splits, bool plan_mode, W4Cfg* cfg, int* tile_end) {
  int64_t n_total = 0;
  for (int g = 0; g < n_members; ++g) n_total += N[g];
  SPECQ_REQUIRE(n_total <= INT32_MAX, SPECQ_EINVAL, "w4a16_grouped: total N too large");
  int rc = w4_config(layout, m_grid, (int)n_total, K, block_m, block_n, splits, plan_mode, cfg, false);
  if (rc) return rc;
  const int BN = 64 * cfg->rw, BM = cfg->mt * 16;
  int tiles = 0;
  for (int g = 0; g < n_members; ++g) {
    tiles += ceil_div(N[g], BN);
    tile_end[g] = tiles;
  }
  cfg->n_tiles = tiles;
  cfg->units = tiles * cfg->splits;
  cfg->grid = chunked_grid(cfg->units, cfg->m_chunks);
  cfg->ws_partials = cfg->splits > 1 ? align_up((size_t)cfg->m_chunks * tiles * cfg->splits * BM * BN * 4, 256) : 0;
  cfg->ws_counters = cfg->splits > 1 ? kCounterBytes : 0;
  SPECQ_REQUIRE((int64_t)cfg->m_chunks * tiles <= kMaxCounters, SPECQ_ENOTSUP,
                "w4a16_grouped: %d x %d tiles exceed the counter region", cfg->m_chunks, tiles);
  return SPECQ_OK;
}

}  // namespace

int w4a16_attrs(int layout, int m_grid, int N, int K, int block_m, int block_n, int num_warps, int split_k,
                specq_kernel_attrs* out) {
  (void)num_warps;
  W4Cfg cfg;
  const bool plan_mode = (layout & kAttrsPlan) != 0;
  layout &= ~kAttrsPlan;
  int rc = w4_config(layout, m_grid, N, K, block_m, block_n, split_k, plan_mode, &cfg);
  if (rc) return rc;
  hipFuncAttributes fa;
  if (hipFuncGetAttributes(&fa, cfg.fn) != hipSuccess) return fail(SPECQ_EIO, "w4a16: hipFuncGetAttributes failed");
  // The name carries the template arguments exactly as profilers print the kernel symbol.
  if (cfg.family == kW4Plan)
    snprintf(out->name, sizeof(out->name), "specq::w4a16_plan_kernel<%d>", layout);
  else if (cfg.family == kW4Rk)
    snprintf(out->name, sizeof(out->name), "specq::w4a16_rk_kernel<%d, %d, %d>", cfg.mt, cfg.rw, layout);
  else {
    int s = 0, nslot = 0, nsw = 0;
    w4a16_ws_shape(cfg.mt, cfg.rw, layout, &s, &nslot, &nsw);
    snprintf(out->name, sizeof(out->name), "specq::w4a16_ws_kernel<%d, %d, %d, %d, %d, %d>", cfg.mt, cfg.rw, s,
             nslot, nsw, layout);
  }
  out->num_regs = fa.numRegs;
  out->lds_bytes = (int)fa.sharedSizeBytes;
  out->scratch_bytes = (int)fa.localSizeBytes;
  out->threads = cfg.family == kW4Rk ? 256 : kW4WsThreads;
  out->grid = cfg.grid;
  out->block_m = cfg.mt * 16; out->block_n = 64 * cfg.rw; out->num_warps = out->threads / 64;
  out->split_k = cfg.splits;
  return SPECQ_OK;
}

}  // namespace specq

using namespace specq;

extern "C" size_t specq_w4a16_workspace_size(int m_grid, int N, int K, int block_m, int block_n, int num_warps,
                                             int split_k) {
  (void)num_warps;
  return w4_workspace(m_grid, N, K, block_m, block_n, split_k);
}

extern "C" int specq_w4a16(const void* a, int64_t lda, const void* wq, int64_t ldq, int wq_layout, const void* sc,
                           int64_t ld_sc, void* c, int64_t ldc, int M, int N, int K, int group, int grid_m_max,
                           const int32_t* plan, int block_m, int block_n, int num_warps, int split_k, void* workspace,
                           size_t workspace_bytes, void* stream) {
  (void)num_warps;
  clear_error();
  SPECQ_REQUIRE(M >= 0 && N > 0 && K > 0, SPECQ_EINVAL, "w4a16: bad sizes M=%d N=%d K=%d", M, N, K);
  SPECQ_REQUIRE(a && wq && sc && c, SPECQ_EINVAL, "w4a16: null tensor pointer");
  SPECQ_REQUIRE(wq_layout >= 0 && wq_layout <= 2, SPECQ_EINVAL, "w4a16: unknown weight layout %d", wq_layout);
  SPECQ_REQUIRE(group > 0 && K % group == 0, SPECQ_EINVAL, "w4a16: group=%d must divide K=%d", group, K);
  SPECQ_REQUIRE(group % (wq_layout == 0 ? 16 : 32) == 0 && (group & (group - 1)) == 0, SPECQ_ENOTSUP,
                "w4a16: group=%d must be a power of two and a multiple of %d for layout %d", group,
                wq_layout == 0 ? 16 : 32, wq_layout);
  const int64_t row_bytes = wq_layout == 1 ? ldq * 4 : ldq;
  SPECQ_REQUIRE((wq_layout == 2 || row_bytes >= K / 2) && lda >= K && ld_sc >= K / group && ldc >= N, SPECQ_EINVAL,
                "w4a16: row strides must cover a row");
  SPECQ_REQUIRE(grid_m_max == 0 || grid_m_max >= M, SPECQ_EINVAL, "w4a16: grid_m_max=%d < M=%d", grid_m_max, M);
  SPECQ_REQUIRE((uintptr_t)a % 16 == 0 && lda % 8 == 0, SPECQ_ENOTSUP,
                "w4a16: activations need 16-byte aligned rows (lda %% 8 == 0)");
  SPECQ_REQUIRE((uintptr_t)wq % 16 == 0 && (wq_layout == 2 || row_bytes % 16 == 0), SPECQ_ENOTSUP,
                "w4a16: packed weights need 16-byte aligned rows");
  SPECQ_REQUIRE((uintptr_t)sc % 2 == 0, SPECQ_EINVAL, "w4a16: misaligned scales");
  const int m_grid = grid_m_max > 0 ? grid_m_max : M;
  if (m_grid == 0) return SPECQ_OK;
  W4Cfg cfg;
  int rc = w4_config(wq_layout, m_grid, N, K, block_m, block_n, split_k, plan != nullptr, &cfg);
  if (rc) return rc;
  const size_t need = cfg.ws_partials + cfg.ws_counters;
  SPECQ_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), SPECQ_ENOSPC,
                "w4a16: workspace of %zu bytes required, %zu given", need, workspace ? workspace_bytes : 0);
  W4A16Params p;
  p.A = (const _Float16*)a; p.lda = lda; p.Wq = (const uint8_t*)wq; p.ldq = row_bytes;
  p.sc = (const _Float16*)sc; p.ld_sc = ld_sc; p.C = (_Float16*)c; p.ldc = ldc; p.plan = plan;
  p.M = M; p.N = N; p.K = K; p.m_grid = m_grid;
  p.group_shift = __builtin_ctz((unsigned)group);
  p.n_tiles = cfg.n_tiles; p.m_chunks = cfg.m_chunks; p.splits = cfg.splits; p.units = cfg.units;
  p.nblocks = cfg.nblocks; p.bps = cfg.bps; p.ntiles16 = ceil_div(N, 16);
  p.counters = need ? (int32_t*)workspace : nullptr;
  p.partials = need ? (float*)((char*)workspace + kCounterBytes) : nullptr;
  p.vec_store = ((uintptr_t)c % 8 == 0) && (ldc % 4 == 0);
  p.n_grp = 1;
  diag_timeline(&p.tl, &p.tl_cap);
  if (cfg.family == kW4Plan) {
    W4PlanParams pp;
    pp.p = p;
    for (int e = 0; e < kW4PlanRows; ++e) pp.t[e] = cfg.plan_t[e];
    return launch(cfg.fn, cfg.grid, kW4WsThreads, 0, (hipStream_t)stream, &pp);
  }
  return launch(cfg.fn, cfg.grid, cfg.family == kW4Rk ? 256 : kW4WsThreads, 0, (hipStream_t)stream, &p);
}

extern "C" int specq_w4a16_grouped_split(int n_members, const int* N, int K, int split_k) {
  if (n_members < 1 || n_members > kW4MaxGroup || N == nullptr || K <= 0 || K % 128 != 0) return 0;
  for (int g = 0; g < n_members; ++g)
    if (N[g] <= 0) return 0;
  return w4_group_splits(n_members, N, K, split_k);
}

extern "C" size_t specq_w4a16_grouped_workspace_size(int m_grid, int n_members, const int* N, int K, int block_m,
                                                     int block_n, int num_warps, int split_k) {
  (void)num_warps;
  if (n_members < 1 || n_members > kW4MaxGroup || N == nullptr || K <= 0 || K % 128 != 0) return 0;
  for (int g = 0; g < n_members; ++g)
    if (N[g] <= 0) return 0;
  size_t need = 0;
  const int splits = w4_group_splits(n_members, N, K, split_k);
  if (n_members == 1 || splits == 0) {
    for (int g = 0; g < n_members; ++g) need = std::max(need, w4_workspace(m_grid, N[g], K, block_m, block_n, split_k));
    return need;
  }
  for (int plan_mode = 0; plan_mode < 2; ++plan_mode) {
    W4Cfg cfg;
    int tile_end[kW4MaxGroup];
    if (w4_group_config(1, m_grid, n_members, N, K, block_m, block_n, splits, plan_mode != 0, &cfg, tile_end) ==
        SPECQ_OK)
      need = std::max(need, cfg.ws_partials + cfg.ws_counters);
  }
  clear_error();
  return need;
}

extern "C" int specq_w4a16_grouped(const void* a, int64_t lda, int n_members, const void* const* wq,
                                   const int64_t* ldq, int wq_layout, const void* const* sc, const int64_t* ld_sc,
                                   void* const* c, const int64_t* ldc, const int* N, int M, int K, int group,
                                   int grid_m_max, const int32_t* plan, int block_m, int block_n, int num_warps,
                                   int split_k, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  SPECQ_REQUIRE(n_members >= 1 && n_members <= kW4MaxGroup, SPECQ_EINVAL,
                "w4a16_grouped: %d GEMMs (1..%d supported)", n_members, kW4MaxGroup);
  SPECQ_REQUIRE(wq && sc && c && ldc && N && ld_sc && (wq_layout == 2 || ldq), SPECQ_EINVAL,
                "w4a16_grouped: null member array");
  // Every member is checked as its own call would check it (the same entry point with M = 0
  // launches nothing and returns after the checks).
  for (int g = 0; g < n_members; ++g) {
    const int rc = specq_w4a16(a, lda, wq[g], wq_layout == 2 ? 0 : ldq[g], wq_layout, sc[g], ld_sc[g], c[g], ldc[g],
                               0, N[g], K, group, 0, nullptr, block_m, block_n, num_warps, split_k, nullptr, 0,
                               stream);
    if (rc) return rc;
  }
  SPECQ_REQUIRE(M >= 0, SPECQ_EINVAL, "w4a16_grouped: bad M=%d", M);
  SPECQ_REQUIRE(grid_m_max == 0 || grid_m_max >= M, SPECQ_EINVAL, "w4a16_grouped: grid_m_max=%d < M=%d", grid_m_max, M);
  const int m_grid = grid_m_max > 0 ? grid_m_max : M;
  if (m_grid == 0) return SPECQ_OK;
  const int splits = w4_group_splits(n_members, N, K, split_k);
  if (n_members == 1 || splits == 0) {
    // Members whose automatic split counts differ run as one launch each, in order on the
    // stream (the workspace is reused: the last workgroup of a tile resets its counter).
    for (int g = 0; g < n_members; ++g) {
      const int rc = specq_w4a16(a, lda, wq[g], wq_layout == 2 ? 0 : ldq[g], wq_layout, sc[g], ld_sc[g], c[g],
                                 ldc[g], M, N[g], K, group, grid_m_max, plan, block_m, block_n, num_warps, split_k,
                                 workspace, workspace_bytes, stream);
      if (rc) return rc;
    }
    return SPECQ_OK;
  }
  W4Cfg cfg;
  int tile_end[kW4MaxGroup];
  int rc = w4_group_config(wq_layout, m_grid, n_members, N, K, block_m, block_n, splits, plan != nullptr, &cfg,
                           tile_end);
  if (rc) return rc;
  const size_t need = cfg.ws_partials + cfg.ws_counters;
  SPECQ_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), SPECQ_ENOSPC,
                "w4a16_grouped: workspace of %zu bytes required, %zu given", need, workspace ? workspace_bytes : 0);
  auto row_bytes = [&](int g) -> int64_t { return wq_layout == 1 ? ldq[g] * 4 : (wq_layout == 0 ? ldq[g] : 0); };
  auto vec_ok = [&](int g) { return ((uintptr_t)c[g] % 8 == 0) && (ldc[g] % 4 == 0) ? 1 : 0; };
  W4A16Params p;
  p.A = (const _Float16*)a; p.lda = lda; p.Wq = (const uint8_t*)wq[0]; p.ldq = row_bytes(0);
  p.sc = (const _Float16*)sc[0]; p.ld_sc = ld_sc[0]; p.C = (_Float16*)c[0]; p.ldc = ldc[0]; p.plan = plan;
  p.M = M; p.N = N[0]; p.K = K; p.m_grid = m_grid;
  p.group_shift = __builtin_ctz((unsigned)group);
  p.n_tiles = cfg.n_tiles; p.m_chunks = cfg.m_chunks; p.splits = cfg.splits; p.units = cfg.units;
  p.nblocks = cfg.nblocks; p.bps = cfg.bps; p.ntiles16 = ceil_div(N[0], 16);
  p.counters = need ? (int32_t*)workspace : nullptr;
  p.partials = need ? (float*)((char*)workspace + kCounterBytes) : nullptr;
  p.vec_store = vec_ok(0);
  p.n_grp = n_members;
  diag_timeline(&p.tl, &p.tl_cap);
  for (int g = 1; g < kW4MaxGroup; ++g) {
    const bool on = g < n_members;
    p.grp_tile_end[g - 1] = on ? tile_end[g - 1] : 0;
    p.grp_Wq[g - 1] = on ? (const uint8_t*)wq[g] : nullptr;
    p.grp_ldq[g - 1] = on ? row_bytes(g) : 0;
    p.grp_sc[g - 1] = on ? (const _Float16*)sc[g] : nullptr;
    p.grp_ld_sc[g - 1] = on ? ld_sc[g] : 0;
    p.grp_C[g - 1] = on ? (_Float16*)c[g] : nullptr;
    p.grp_ldc[g - 1] = on ? ldc[g] : 0;
    p.grp_N[g - 1] = on ? N[g] : 0;
    p.grp_ntiles16[g - 1] = on ? ceil_div(N[g], 16) : 0;
    p.grp_vec_store[g - 1] = on ? vec_ok(g) : 0;
  }
  return launch(cfg.fn, cfg.grid, cfg.family == kW4Rk ? 256 : kW4WsThreads, 0, (hipStream_t)stream, &p);
}

extern "C" size_t specq_w4a16_packed_bytes(int N, int K) {
  if (N <= 0 || K <= 0 || K % 128 != 0) return 0;
  return (size_t)ceil_div(N, 16) * (K / 128) * 1024;
}

extern "C" int specq_w4a16_pack_weight(const void* wq, int64_t ldq, int wq_layout, int N, int K, void* packed,
                                       void* stream) {
  clear_error();
  SPECQ_REQUIRE(wq && packed, SPECQ_EINVAL, "w4a16_pack_weight: null tensor pointer");
  SPECQ_REQUIRE(wq_layout == 0 || wq_layout == 1, SPECQ_EINVAL, "w4a16_pack_weight: layout %d is not 0 or 1",
                wq_layout);
  SPECQ_REQUIRE(N > 0 && K > 0 && K % 128 == 0, SPECQ_ENOTSUP, "w4a16_pack_weight: K=%d must be a multiple of 128", K);
  const int64_t row_bytes = wq_layout == 1 ? ldq * 4 : ldq;
  SPECQ_REQUIRE(row_bytes >= K / 2, SPECQ_EINVAL, "w4a16_pack_weight: row stride %lld too small", (long long)ldq);
  SPECQ_REQUIRE((uintptr_t)packed % 16 == 0, SPECQ_EINVAL, "w4a16_pack_weight: misaligned output");
  const int64_t frags = (int64_t)ceil_div(N, 16) * (K / 128);
  SPECQ_REQUIRE(ceil_div64(frags, 4) <= INT32_MAX, SPECQ_ENOTSUP, "w4a16_pack_weight: weight too large");
  const uint8_t* w = (const uint8_t*)wq;
  void* args[] = {(void*)&w, (void*)&row_bytes, (void*)&wq_layout, (void*)&N, (void*)&K, (void*)&packed};
  hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&w4a16_pack_kernel),
                                 dim3((unsigned)ceil_div64(frags, 4)), dim3(256), args, 0, (hipStream_t)stream);
  if (e != hipSuccess) {
    set_error("w4a16_pack_weight: hipLaunchKernel failed: %s", hipGetErrorString(e));
    return SPECQ_EIO;
  }
  return SPECQ_OK;
}
