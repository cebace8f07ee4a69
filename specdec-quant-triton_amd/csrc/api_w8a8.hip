// C ABI for the W8A8 GEMM: argument validation, kernel-family and tile selection, launch.
//
// Kernel families (all compute identical INT32 sums, so every choice is bit-identical):
//   RK      direct-activation streaming kernel (w8a8_rk.hpp) for 16-row token tiles: weights
//           and activations go straight from memory into MFMA operand registers.
//   WS      weight streaming with LDS-staged activations (w8a8_ws.hpp) for deeper token tiles.
//   LEGACY  register-pipelined kernel with 16/8/4/1-byte loads (w8a8.hpp): any alignment.
// RK and WS read the row-major weight or the packed K-step-major fragments and need 16-byte
// aligned activation rows.  Weight layout 2 is the packed INT4 weight of W4A8 (INT4 weights on
// the INT8 MFMA path with a per-channel scale in the epilogue), served by the RK and WS
// families with the same tiles.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <map>
#include <mutex>
#include <vector>

#include "api_common.hpp"
#include "w8a8.hpp"
#include "w8a8_plan.hpp"
#include "w8a8_tiles.hpp"

namespace specq {

const void* w8a8_kernel_rw1(int mt, int vec);
const void* w8a8_plan_fn_l0(int variant);
const void* w8a8_plan_fn_l1(int variant);
const void* w8a8_plan_fn_l2(int variant);
const void* w8a8_kernel_rw2(int mt, int vec);
const void* w8a8_kernel_rw4(int mt, int vec);

// Packs a row-major int8 weight [N, K] (row stride ldw) into MFMA fragments stored K-step-major:
// packed[s][t][l*16 + b] = W[16t + l%16][64s + 16*(l/16) + b], zero-padded to whole tiles,
// with s the 64-byte K step and t the 16-row tile (ntiles = ceil(N/16) tiles per step).
__global__ __launch_bounds__(256) void w8a8_pack_kernel(const int8_t* __restrict__ W, int64_t ldw, int N, int K,
                                                        int8_t* __restrict__ out) {
  const int ksteps = (K + 63) / 64;
  const int ntiles = (N + 15) / 16;
  const int64_t frag = blockIdx.x * 4 + (threadIdx.x >> 6);  // one wave per fragment
  if (frag >= (int64_t)ntiles * ksteps) return;
  const int s = (int)(frag / ntiles), t = (int)(frag % ntiles);
  const int l = threadIdx.x & 63;
  const int row = 16 * t + (l & 15), k0 = 64 * s + 16 * (l >> 4);
  int w4[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int v = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int k = k0 + 4 * i + b;
      const int x = (row < N && k < K) ? (int)(uint8_t)W[(int64_t)row * ldw + k] : 0;
      v |= x << (8 * b);
    }
    w4[i] = v;
  }
  *reinterpret_cast<v4i*>(out + frag * 1024 + l * 16) = v4i{w4[0], w4[1], w4[2], w4[3]};
}

// Packs an INT4 weight (reference uint8 layout 0 or int32 layout 1, nibbles with offset 8) into
// the W4A8 fragments: fragment (s, t) of 64-wide K step s and 16-row tile t is the 512 bytes at
// (s * ntiles + t) * 512; lane l's dword d, byte i holds the two's-complement nibbles of
// w[16t + l%16][64s + 16*(l/16) + 8d + i] (low) and [... + 8d + 4 + i] (high), zero past N or K.
__global__ __launch_bounds__(256) void w4a8_pack_kernel(const uint8_t* __restrict__ q, int64_t ldq, int layout, int N,
                                                        int K, int8_t* __restrict__ out) {
  const int ksteps = (K + 63) / 64;
  const int ntiles = (N + 15) / 16;
  const int64_t frag = blockIdx.x * 4 + (threadIdx.x >> 6);  // one wave per fragment
  if (frag >= (int64_t)ntiles * ksteps) return;
  const int s = (int)(frag / ntiles), t = (int)(frag % ntiles);
  const int l = threadIdx.x & 63;
  const int row = 16 * t + (l & 15), k0 = 64 * s + 16 * (l >> 4);
  auto nib = [&](int k) -> uint32_t {  // two's-complement nibble of (row, k); 0 outside the weight
    if (row >= N || k >= K) return 0u;
    uint32_t n;
    if (layout == 0) {  // byte j of a row: k = j (low nibble), k = j + K/2 (high nibble)
      const int half = K / 2;
      const uint32_t b = q[(int64_t)row * ldq + (k < half ? k : k - half)];
      n = k < half ? (b & 0xFu) : (b >> 4);
    } else {  // int32 word j of a row: nibble i holds k = 8j + i
      const uint32_t w = reinterpret_cast<const uint32_t*>(q)[(int64_t)row * ldq + k / 8];
      n = (w >> (4 * (k % 8))) & 0xFu;
    }
    return n ^ 8u;  // offset-8 nibble -> two's complement
  };
  uint32_t d[2];
#pragma unroll
  for (int dd = 0; dd < 2; ++dd) {
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) v |= (nib(k0 + 8 * dd + i) | (nib(k0 + 8 * dd + 4 + i) << 4)) << (8 * i);
    d[dd] = v;
  }
  *reinterpret_cast<v2i*>(out + frag * 512 + l * 8) = v2i{(int)d[0], (int)d[1]};
}

// Device scratch of the allocation-free entry point specq_w8a8_packed_noalloc: the split-K
// counters (the first kCounterBytes) and the INT32 partial tiles.  Each GPU the library runs on
// holds its own copy until the process ends.  In host code `scratch` is only a stand-in for
// the symbol: its device address on a GPU comes from hipGetSymbolAddress with that GPU current.
static __device__ __align__(256) uint8_t scratch[SPECQ_NOALLOC_SCRATCH_BYTES];
static_assert(SPECQ_NOALLOC_SCRATCH_BYTES > kCounterBytes, "scratch holds the counter region");

// Zeroes n int32 counters (a fill kernel, not a memset node, so the call may be captured).
__global__ __launch_bounds__(256) void zero_i32_kernel(int32_t* __restrict__ p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Device address of `scratch` on the current GPU, looked up once per GPU.
static int noalloc_scratch(void** out) {
  static std::mutex mu;
  static std::vector<void*> ptrs;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return fail(SPECQ_EIO, "w8a8_packed_noalloc: no current device");
  std::lock_guard<std::mutex> lock(mu);
  if ((int)ptrs.size() <= dev) ptrs.resize(dev + 1, nullptr);
  if (ptrs[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error("w8a8_packed_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
      return SPECQ_EIO;
    }
    ptrs[dev] = ptr;
  }
  *out = ptrs[dev];
  return SPECQ_OK;
}

// Kernel family override (0 = automatic), set through specq_set_option("w8a8_path", v).
std::atomic<int> g_w8a8_path{0};
extern std::atomic<int> g_w4a16_path;  // api_w4a16.hip
extern std::atomic<int> g_attn_target;  // api_attn.hip
extern std::atomic<int> g_tuned_tiles;  // api_common.hip

namespace {

// kPlan: plan-mode launch holding the menu of RK / WS tilings (w8a8_plan.hpp), one per 16 rows
// of the active M.
enum Family { kRk = 1, kWs = 2, kLegacy = 3, kPlan = 4 };

struct W8A8Cfg {
  int family, layout;
  int mt, rw, nw, vec, splits, k_range, n_tiles, m_chunks;
  int bn;         // channels per workgroup
  int bnsel;      // RK/WS channel-width variant (0..3 for 16/32/64/128)
  size_t lds, ws_partials, ws_counters;
  const void* fn;
  // kPlan: the tiling of each 16-row step of M, the grid (the largest tiling's) and the
  // counters the largest tiling uses; mt / bn / splits above describe the entry of M = m_grid.
  W8A8PlanTile plan_t[kW8A8PlanRows];
  int plan_grid, n_counters;
};

int round_mt_for_vec(int mt, int vec, int rw) {
  if (vec == 16) return mt;
  static const int avail[] = {1, 2, 4, 8, 16, 20};
  for (int a : avail)
    if (a >= mt && a * rw <= 40) return a;
  return -1;
}

const void* legacy_fn(int mt, int rw, int vec) {
  switch (rw) {
    case 1: return w8a8_kernel_rw1(mt, vec);
    case 2: return w8a8_kernel_rw2(mt, vec);
    case 4: return w8a8_kernel_rw4(mt, vec);
  }
  return nullptr;
}

const void* ws_fn(int bnsel, int layout, int mt) {
  switch (bnsel * 3 + layout) {
    case 0: return w8a8_ws_fn_n16_l0(mt);
    case 1: return w8a8_ws_fn_n16_l1(mt);
    case 2: return w8a8_ws_fn_n16_l2(mt);
    case 3: return w8a8_ws_fn_n32_l0(mt);
    case 4: return w8a8_ws_fn_n32_l1(mt);
    case 5: return w8a8_ws_fn_n32_l2(mt);
    case 6: return w8a8_ws_fn_n64_l0(mt);
    case 7: return w8a8_ws_fn_n64_l1(mt);
    case 8: return w8a8_ws_fn_n64_l2(mt);
    case 9: return w8a8_ws_fn_n128_l0(mt);
    case 10: return w8a8_ws_fn_n128_l1(mt);
    case 11: return w8a8_ws_fn_n128_l2(mt);
  }
  return nullptr;
}

int bn_of_sel(int sel) { return 16 << sel; }
int kw_of_sel(int sel) { return sel == 0 ? 4 : (sel == 1 ? 2 : 1); }  // waves splitting K

// Channel block and split count of the LDS-staged kernel from a cost model fitted to measured
// latencies of the Llama-3-8B linears (qkv, o, gate_up, down, gate, k/v at M = 24..288; mean
// regret 0.6%, worst 5.5% against the best measured tile): a workgroup streams
// (BN + rows) * K / splits bytes at ~50 GB/s per CU, all weights cross HBM at ~7 TB/s, and a
// split costs ~2 us plus writing and reading its INT32 partial tiles at ~2 TB/s.  Shapes that
// need more workgroups than CUs are left out (one workgroup per CU streams best).
// `bnsel_fixed` >= 0 keeps the caller's BLOCK_N; `splits_fixed` > 0 keeps its split count.
// `wb` is the weight bytes per element (1 for INT8, 0.5 for the INT4 weights of W4A8).
void ws_auto_tiles(int rows, int m_chunks, int N, int K, double wb, int bnsel_fixed, int splits_fixed, int* bnsel,
                   int* splits) {
  const int cus = device_cus();
  const int mpad = ceil_div(rows, 16) * 16;
  double best_t = 0;
  int best_sel = -1, best_s = 1;
  for (int pass = 0; pass < 2 && best_sel < 0; ++pass) {  // pass 1 only if nothing fits the CUs
    for (int sel = 0; sel < 4; ++sel) {
      if (bnsel_fixed >= 0 && sel != bnsel_fixed) continue;
      const int bn = bn_of_sel(sel);
      const int cand[3] = {splits_fixed > 0 ? splits_fixed : 1, 2, 4};
      for (int ci = 0; ci < (splits_fixed > 0 ? 1 : 3); ++ci) {
        const int s = cand[ci];
        if (pass == 0 && (int64_t)ceil_div(N, bn) * s * m_chunks > cus) continue;
        double t = std::max((bn * wb + rows) * K / s / 50e3, N * wb * K / 7e6);
        if (s > 1) t += 2.0 + (double)s * mpad * N * 8 / 2e6;
        if (pass == 1) t *= (double)ceil_div(ceil_div(N, bn) * s * m_chunks, cus);  // rounds of workgroups
        if (best_sel < 0 || t < best_t) { best_t = t; best_sel = sel; best_s = s; }
      }
    }
  }
  *bnsel = best_sel;
  *splits = best_s;
}
static_assert(W8A8BnSel<0>::KW == 4 && W8A8BnSel<1>::KW == 2 && W8A8BnSel<2>::KW == 1 && W8A8BnSel<3>::KW == 1,
              "kw_of_sel mirrors the tile table");

// Eager tile choice over the token-tile depth as well: M is cut into c = 1..6 chunks of
// mt = ceil(rows16 / c) 16-row tiles, and each (mt, channel block, split count) is priced by
// a model fitted to a sweep of 3,600 measured tiles (qkv, o, gate_up, down, gate, k/v at
// M = 17..300; mean regret 0.85% against the best measured tile, where a single chunk over
// all of M lost up to 48% at M >= 128):
//   t = max(rounds * (BN * wb + rows) * K / s / 45 GB/s, N * wb * K / 6 TB/s) + 1 us
//       (+ 2 us and the INT32 partial tiles at 2 TB/s when s > 1),
// with rounds = ceil(workgroups / CUs): a CU pulls its workgroups' activation chunks and
// weight tiles at ~45 GB/s, and the weight re-reads of later M chunks come from L2 / MALL.
// 16-row chunks run on the direct-activation kernel, measured fast only with 16-channel
// blocks, no split and one round of workgroups.
// Modelled time of one tiling (token-tile depth mt, channel block sel, requested split count)
// of `rows16` 16-row token tiles on `cus` CUs, from the model above; negative when the tiling
// is not one the model allows.  *s_eff is the split count after whole-chunk boundaries.
double w8a8_model_time(int rows16, int N, int K, double wb, int mt, int sel, int s_req, int cus, int* s_eff) {
  const int ksteps = ceil_div(K, 64), kq = ceil_div(ksteps, 4);
  const int chunks = ceil_div(rows16, mt), rows = mt * 16;
  const int bn = bn_of_sel(sel);
  int s = std::min(s_req, kq);
  s = ceil_div(K, ceil_div(kq, s) * 256);  // split count after whole-chunk boundaries
  const int64_t wgs = (int64_t)ceil_div(N, bn) * s * chunks;
  if (mt == 1 && (sel != 0 || s != 1 || wgs > cus)) return -1.0;
  const double rounds = (double)ceil_div((int)wgs, cus);
  double t = std::max(rounds * (bn * wb + rows) * K / s / 45e3, N * wb * K / 6e6) + 1.0;
  if (s > 1) t += 2.0 + (double)s * rows * chunks * N * 8 / 2e6;
  *s_eff = s;
  return t;
}

void w8a8_auto_tiles(int M, int N, int K, double wb, int bnsel_fixed, int splits_fixed, int* mt_out, int* bnsel,
                     int* splits) {
  const int rows16 = ceil_div(std::max(M, 1), 16);
  const int cus = device_cus();
  double best_t = 0;
  int best_mt = -1, best_sel = 2, best_s = 1, last_mt = -1;
  const int max_c = std::max(6, ceil_div(rows16, kW8A8MaxMt));  // past 6 chunks only when M needs it
  for (int c = 1; c <= max_c; ++c) {
    const int mt = ceil_div(rows16, c);
    if (mt == last_mt || mt > kW8A8MaxMt) continue;
    last_mt = mt;
    for (int sel = 0; sel < 4; ++sel) {
      if (bnsel_fixed >= 0 && sel != bnsel_fixed) continue;
      const int cand[3] = {splits_fixed > 0 ? splits_fixed : 1, 2, 4};
      for (int ci = 0; ci < (splits_fixed > 0 ? 1 : 3); ++ci) {
        int s = 1;
        const double t = w8a8_model_time(rows16, N, K, wb, mt, sel, cand[ci], cus, &s);
        if (t < 0) continue;
        // Equal prices go to the shallower token tile (fewer activation rows per workgroup).
        const bool tie = best_mt >= 0 && std::fabs(t - best_t) <= 1e-9 * best_t;
        if (best_mt < 0 || (t < best_t && !tie) || (tie && mt < best_mt)) {
          best_t = t; best_mt = mt; best_sel = sel; best_s = s;
        }
      }
    }
  }
  *mt_out = best_mt;
  *bnsel = best_sel;
  *splits = best_s;
}

// Resolve the kernel and its tiles.  `vec` is the operand alignment (16 when unknown),
// `layout` 0 = row-major weight, 1 = packed fragments.
int w8a8_config(int layout, int m_grid, int N, int K, int block_m, int block_n, int num_warps, int split_k,
                int vec, bool plan_mode, W8A8Cfg* cfg) {
  SPECQ_REQUIRE(m_grid >= 0 && N > 0 && K > 0, SPECQ_EINVAL, "w8a8: bad sizes M=%d N=%d K=%d", m_grid, N, K);
  SPECQ_REQUIRE(block_n == 0 || block_n == 16 || block_n == 32 || block_n == 64 || block_n == 128, SPECQ_ENOTSUP,
                "w8a8: BLOCK_N=%d must be 16, 32, 64 or 128", block_n);
  const int rows16 = ceil_div(m_grid > 0 ? m_grid : 1, 16);
  const int want = block_n > 0 ? (block_n == 16 ? 0 : (block_n == 32 ? 1 : (block_n == 64 ? 2 : 3))) : -1;
  const int path = g_w8a8_path.load();
  // Plan-mode calls with automatic tiles get the launch that picks a tiling per 16 rows of the
  // active M on the device (its table is filled by w8a8_plan_table for the launch's GEMMs).
  if (plan_mode && block_m <= 0 && block_n <= 0 && split_k <= 0 && vec == 16 && path == 0) {
    cfg->family = kPlan; cfg->layout = layout; cfg->vec = vec; cfg->nw = 4; cfg->rw = 1;
    return SPECQ_OK;
  }
  // Eager calls with automatic tiles on a launch shape of the measured table run its tile;
  // other eager calls with an automatic BLOCK_M on the streaming kernels choose the token-tile
  // depth, channel block and split count together from the cost model.
  int t_bm = 0, t_bn = 0, t_sk = 0;
  const bool tuned = block_m <= 0 && block_n <= 0 && split_k <= 0 && !plan_mode && vec == 16 && path == 0 &&
                     layout != 2 && tuned_tile(0, N, K, std::max(m_grid, 1), &t_bm, &t_bn, &t_sk);
  const bool joint = !tuned && block_m <= 0 && !plan_mode && vec == 16 && path == 0 && rows16 > 1;
  int joint_sel = -1, joint_splits = 1;
  int mt;
  if (tuned) {
    mt = t_bm / 16;
    joint_sel = t_bn == 16 ? 0 : (t_bn == 32 ? 1 : (t_bn == 64 ? 2 : 3));
    joint_splits = t_sk;
  } else if (joint) {
    w8a8_auto_tiles(m_grid, N, K, layout == 2 ? 0.5 : 1.0, want, split_k, &mt, &joint_sel, &joint_splits);
  } else if (block_m > 0) {
    SPECQ_REQUIRE(block_m % 16 == 0 && block_m <= 16 * kW8A8MaxMt, SPECQ_ENOTSUP,
                  "w8a8: BLOCK_M=%d must be a multiple of 16 and at most %d", block_m, 16 * kW8A8MaxMt);
    mt = block_m / 16;
  } else {
    // One chunk of token rows covering M (the weight is then read once), split evenly when
    // M exceeds the deepest tile.  With a plan the grid covers the largest M while the
    // active M is usually much smaller: chunks of at most 80 rows then let the chunks past
    // the active M exit at once instead of running a full-depth tile.
    const int cap = plan_mode ? 5 : kW8A8MaxMt;
    const int chunks = ceil_div(rows16, cap);
    mt = ceil_div(rows16, chunks);
  }
  int family;
  if (vec != 16) family = kLegacy;
  else if (path == kLegacy && layout == 0) family = kLegacy;
  else if (path == kRk) family = kRk;
  else if (path == kWs && mt >= 2) family = kWs;
  else family = mt == 1 ? kRk : kWs;

  int nw = 4, rw = 1, bnsel = 2, ws_splits = 1;
  const void* fn = nullptr;
  if (family == kRk || family == kWs) {
    if (joint || tuned) {
      bnsel = joint_sel;
      ws_splits = joint_splits;
    } else if (family == kWs) {
      // With a plan the grid is sized for the largest M, but usually one M-chunk is active.
      const int rows = std::min(std::max(m_grid, 1), mt * 16);
      const int chunks = plan_mode ? 1 : ceil_div(std::max(m_grid, 1), mt * 16);
      ws_auto_tiles(rows, chunks, N, K, layout == 2 ? 0.5 : 1.0, want, split_k, &bnsel, &ws_splits);
    } else if (want >= 0) {
      bnsel = want;
    } else {
      // Measured on the Llama-3-8B linears at M = 1..16: the narrowest channel block whose
      // workgroups fit the CUs in one round streams best (16 channels for o/down/k/v, 32 for
      // qkv, 64 for gate, 128 for the fused gate_up), without splitting K.
      const int chunks = ceil_div(std::max(m_grid, 1), 16);
      bnsel = 3;
      for (int sel = 0; sel < 3; ++sel)
        if ((int64_t)ceil_div(N, bn_of_sel(sel)) * chunks <= device_cus()) { bnsel = sel; break; }
    }
    if (family == kRk) {
      if (mt > 1) {
        // The direct-activation kernel holds one 16-row token tile: deeper BLOCK_M requests
        // are served as several 16-row chunks.
        mt = 1;
      }
      fn = w8a8_rk_fn(bnsel, layout);
    } else {
      fn = ws_fn(bnsel, layout, mt);
    }
  }
  if (family == kLegacy) {
    rw = block_n > 0 ? (block_n >= 64 ? 4 : block_n / 16) : (N <= 16 ? 1 : 2);
    while (rw > 1 && rw * mt > 40) rw >>= 1;
    int mt_eff = round_mt_for_vec(mt, vec, rw);
    if (mt_eff < 0 && rw > 1) { rw = 1; mt_eff = round_mt_for_vec(mt, vec, rw); }
    SPECQ_REQUIRE(mt_eff > 0, SPECQ_ENOTSUP, "w8a8: no kernel for BLOCK_M=%d at %d-byte alignment", mt * 16, vec);
    mt = mt_eff;
    nw = num_warps <= 0 ? 4 : (num_warps >= 4 ? 4 : (num_warps >= 2 ? 2 : 1));
    fn = legacy_fn(mt, rw, vec);
  }
  SPECQ_REQUIRE(fn != nullptr, SPECQ_ENOTSUP, "w8a8: no kernel for BLOCK_M=%d BLOCK_N=%d", mt * 16, block_n);

  cfg->family = family; cfg->layout = layout; cfg->fn = fn;
  cfg->mt = mt; cfg->rw = rw; cfg->nw = nw; cfg->vec = vec; cfg->bnsel = bnsel;
  cfg->bn = family == kLegacy ? rw * 16 : bn_of_sel(bnsel);
  cfg->n_tiles = ceil_div(N, cfg->bn);
  cfg->m_chunks = ceil_div(m_grid > 0 ? m_grid : 1, mt * 16);
  const int BM = mt * 16, BN = cfg->bn;
  if (family == kRk) {
    cfg->lds = (size_t)(kw_of_sel(bnsel) - 1) * BM * BN * 4;  // one reduction slice per non-owner wave
  } else if (family == kWs) {
    cfg->lds = 0;  // static LDS
  } else {
    cfg->lds = nw > 1 ? (size_t)BM * (BN + kW8A8Pad) * 4 : 0;
  }

  const int ksteps = ceil_div(K, 64);
  int splits;
  if (split_k > 0) {
    splits = split_k;
  } else if (tuned) {
    splits = t_sk;
  } else if (family == kLegacy) {
    const int target = 2 * device_cus();
    const int base = cfg->n_tiles * cfg->m_chunks;
    splits = 4 * base >= 3 * target ? 1 : ceil_div(target, base);
    const int max_splits = std::max(1, ksteps / (2 * nw));
    splits = std::min(splits, max_splits);
  } else if (family == kWs) {
    splits = ws_splits;
  } else {
    splits = 1;
  }
  // Split boundaries on whole 256-byte blocks (one activation chunk of the streaming kernels).
  const int quantum = family == kLegacy ? 1 : 4;
  const int kq = ceil_div(ksteps, quantum);
  if (splits > kq) splits = kq;
  if (splits < 1) splits = 1;
  const int k_range = ceil_div(kq, splits) * quantum * 64;
  splits = ceil_div(K, k_range);
  cfg->splits = splits;
  cfg->k_range = k_range;
  cfg->ws_partials = splits > 1 ? align_up((size_t)cfg->m_chunks * cfg->n_tiles * splits * BM * BN * 4, 256) : 0;
  cfg->ws_counters = splits > 1 ? kCounterBytes : 0;
  SPECQ_REQUIRE((int64_t)cfg->m_chunks * cfg->n_tiles <= kMaxCounters, SPECQ_ENOTSUP,
                "w8a8: %d x %d tiles exceed the counter region", cfg->m_chunks, cfg->n_tiles);
  return SPECQ_OK;
}

// The GEMMs of one launch: one, or up to kW8A8MaxGroup sharing the activation (a grouped launch).
struct W8A8Group {
  int n;
  const void* w[kW8A8MaxGroup];
  int64_t ldw[kW8A8MaxGroup];
  const float* sw[kW8A8MaxGroup];
  void* c[kW8A8MaxGroup];
  int64_t ldc[kW8A8MaxGroup];
  int N[kW8A8MaxGroup];
  int n_total() const {
    int t = 0;
    for (int g = 0; g < n; ++g) t += N[g];
    return t;
  }
};

W8A8Group single(const void* w, int64_t ldw, const float* sw, void* c, int64_t ldc, int N) {
  W8A8Group g;
  g.n = 1; g.w[0] = w; g.ldw[0] = ldw; g.sw[0] = sw; g.c[0] = c; g.ldc[0] = ldc; g.N[0] = N;
  return g;
}

// The per-16-row table of the plan-mode launch: for each step of the active M, the menu
// tiling and split count the eager cost model prices lowest at the step's largest M (the
// decode rule of eager calls at M <= 16), with its channel tiles counted per GEMM of the group.
int w8a8_plan_table(int m_grid, const W8A8Group& grp, int K, W8A8Cfg* cfg) {
  // Tables are cached per (device CUs, layout, grid, K, member widths): building one prices
  // a few thousand tilings, and plan-mode calls repeat the same shapes.
  const int cus = device_cus();
  struct Key {
    int v[9];
    bool operator<(const Key& o) const { return std::lexicographical_compare(v, v + 9, o.v, o.v + 9); }
  };
  Key key{{cus, cfg->layout, m_grid, K, grp.n, grp.N[0], grp.n > 1 ? grp.N[1] : 0, grp.n > 2 ? grp.N[2] : 0,
           grp.n > 3 ? grp.N[3] : 0}};
  static std::mutex mu;
  static std::map<Key, W8A8Cfg> cache;
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) {
      *cfg = it->second;
      return SPECQ_OK;
    }
  }
  const int N = grp.n_total();
  const double wb = cfg->layout == 2 ? 0.5 : 1.0;
  const int R = ceil_div(std::max(m_grid, 1), 16);
  const int ksteps = ceil_div(K, 64), kq = ceil_div(ksteps, 4);
  // Menu entry and split count of each step, per launch variant, and the variant whose steps
  // the model prices lower in total (ties to variant 0, the smaller LDS footprint).
  int pick[2][kW8A8PlanRows], split_of[2][kW8A8PlanRows];
  double total[2] = {0, 0};
  for (int v = 0; v < 2; ++v) {
    for (int e = 0; e < kW8A8PlanRows; ++e) {
      const int r = e == kW8A8PlanRows - 1 ? R : std::min(e + 1, R);
      int path = -1, s = 1;
      double best = 0;
      int64_t best_wgs = 0;
      if (r == 1) {
        int sel = 3;
        for (int c = 0; c < 3; ++c)
          if (ceil_div(N, bn_of_sel(c)) <= cus) { sel = c; break; }
        path = sel;  // menu entries 0..3: the direct-activation tile of channel block sel
      } else {
        for (int i = 0; i < kW8A8PlanMenu; ++i) {
          for (int s_req : {1, 2, 4}) {
            int se = 1;
            const int mt_i = kW8A8PlanMenuMt[v][i];
            const double t = w8a8_model_time(r, N, K, wb, mt_i, kW8A8PlanMenuSel[v][i], s_req, cus, &se);
            if (t < 0) continue;
            // Equal prices go to fewer workgroups (a plan-mode launch holds one workgroup per CU,
            // so every round counts), then to the shallower token tile.
            const int64_t wgs = (int64_t)ceil_div(N, bn_of_sel(kW8A8PlanMenuSel[v][i])) * se * ceil_div(r, mt_i);
            const bool tie = path >= 0 && std::fabs(t - best) <= 1e-9 * best;
            if (path < 0 || (t < best && !tie) ||
                (tie && (wgs < best_wgs || (wgs == best_wgs && mt_i < kW8A8PlanMenuMt[v][path])))) {
              best = t; path = i; s = se; best_wgs = wgs;
            }
          }
        }
      }
      SPECQ_REQUIRE(path >= 0, SPECQ_ENOTSUP, "w8a8 plan: no tiling for M=%d N=%d K=%d", 16 * r, N, K);
      pick[v][e] = path;
      split_of[v][e] = s;
      if (e < R) total[v] += best;
    }
  }
  const int v = total[1] < total[0] ? 1 : 0;
  cfg->fn = cfg->layout == 0 ? w8a8_plan_fn_l0(v) : (cfg->layout == 1 ? w8a8_plan_fn_l1(v) : w8a8_plan_fn_l2(v));
  size_t ws = 0;
  int grid = 0, n_ctr = 0;
  size_t lds = 0;
  for (int e = 0; e < kW8A8PlanRows; ++e) {
    const int r = e == kW8A8PlanRows - 1 ? R : std::min(e + 1, R);
    const int path = pick[v][e];
    int s = split_of[v][e];
    const int mt = kW8A8PlanMenuMt[v][path], bn = bn_of_sel(kW8A8PlanMenuSel[v][path]);
    W8A8PlanTile& t = cfg->plan_t[e];
    t.path = path;
    t.m_chunks = ceil_div(r, mt);
    int tiles = 0;
    for (int g = 0; g < grp.n; ++g) {
      tiles += ceil_div(grp.N[g], bn);
      if (g + 1 < grp.n) t.grp_tile_end[g] = tiles;
    }
    for (int g = grp.n - 1; g < 3; ++g) t.grp_tile_end[g] = tiles;
    t.n_tiles = tiles;
    s = std::min(std::max(s, 1), kq);
    t.k_range = ceil_div(kq, s) * 4 * 64;
    t.splits = ceil_div(K, t.k_range);
    SPECQ_REQUIRE((int64_t)t.m_chunks * tiles <= kMaxCounters, SPECQ_ENOTSUP,
                  "w8a8 plan: %d x %d tiles exceed the counter region", t.m_chunks, tiles);
    if (t.splits > 1) {
      ws = std::max(ws, align_up((size_t)t.m_chunks * tiles * t.splits * (mt * 16) * bn * 4, 256));
      n_ctr = std::max(n_ctr, t.m_chunks * tiles);
    }
    grid = std::max(grid, chunked_grid(tiles * t.splits, t.m_chunks));
    if (mt == 1) lds = std::max(lds, (size_t)(kw_of_sel(kW8A8PlanMenuSel[v][path]) - 1) * 16 * bn * 4);
  }
  const W8A8PlanTile& top = cfg->plan_t[std::min(R, kW8A8PlanRows) - 1];
  cfg->mt = kW8A8PlanMenuMt[v][top.path];
  cfg->bnsel = kW8A8PlanMenuSel[v][top.path];
  cfg->bn = bn_of_sel(cfg->bnsel);
  cfg->n_tiles = top.n_tiles; cfg->m_chunks = top.m_chunks; cfg->splits = top.splits; cfg->k_range = top.k_range;
  cfg->ws_partials = ws;
  cfg->ws_counters = n_ctr > 0 ? kCounterBytes : 0;
  cfg->n_counters = n_ctr;
  cfg->plan_grid = grid;
  cfg->lds = lds;
  std::lock_guard<std::mutex> lock(mu);
  cache[key] = *cfg;
  return SPECQ_OK;
}

// Tiles of a grouped launch: chosen as for one GEMM of the members' total width, then every
// member gets whole channel blocks of its own (its last block may be partial).
int w8a8_group_config(int layout, int m_grid, const W8A8Group& grp, int K, int block_m, int block_n, int num_warps,
                      int split_k, int vec, bool plan_mode, W8A8Cfg* cfg) {
  int rc = w8a8_config(layout, m_grid, grp.n_total(), K, block_m, block_n, num_warps, split_k, vec, plan_mode, cfg);
  if (rc) return rc;
  if (cfg->family == kPlan) return w8a8_plan_table(m_grid, grp, K, cfg);
  if (grp.n == 1) return rc;
  SPECQ_REQUIRE(cfg->family != kLegacy, SPECQ_ENOTSUP,
                "w8a8 grouped: needs 16-byte aligned operands and K %% 16 == 0 (the streaming kernels)");
  int tiles = 0;
  for (int g = 0; g < grp.n; ++g) tiles += ceil_div(grp.N[g], cfg->bn);
  cfg->n_tiles = tiles;
  cfg->ws_partials =
      cfg->splits > 1 ? align_up((size_t)cfg->m_chunks * tiles * cfg->splits * (cfg->mt * 16) * cfg->bn * 4, 256) : 0;
  SPECQ_REQUIRE((int64_t)cfg->m_chunks * tiles <= kMaxCounters, SPECQ_ENOTSUP,
                "w8a8: %d x %d tiles exceed the counter region", cfg->m_chunks, tiles);
  return SPECQ_OK;
}

// With `static_scratch` the call runs on the device scratch array instead of a caller workspace:
// it is refused when it needs more than that array holds, and the counters it uses are zeroed
// (on the stream, before the GEMM) rather than assumed zero.
int run_w8a8(int layout, const int8_t* a, int64_t lda, const W8A8Group& grp, const float* sa, int M, int K,
             int grid_m_max, const int32_t* plan, int block_m, int block_n, int num_warps, int split_k,
             void* workspace, size_t workspace_bytes, void* stream, bool static_scratch = false) {
  SPECQ_REQUIRE(grp.n >= 1 && grp.n <= kW8A8MaxGroup, SPECQ_EINVAL, "w8a8: %d GEMMs in a group (1..%d)", grp.n,
                kW8A8MaxGroup);
  SPECQ_REQUIRE(M >= 0 && K > 0, SPECQ_EINVAL, "w8a8: bad sizes M=%d K=%d", M, K);
  SPECQ_REQUIRE(a && sa && lda >= K, SPECQ_EINVAL, "w8a8: null activation pointer or lda=%lld < K", (long long)lda);
  int vec = common_vec({(uint64_t)(uintptr_t)a, (uint64_t)lda, (uint64_t)K});
  for (int g = 0; g < grp.n; ++g) {
    const int N = grp.N[g];
    SPECQ_REQUIRE(N > 0, SPECQ_EINVAL, "w8a8: bad sizes M=%d N=%d K=%d", M, N, K);
    SPECQ_REQUIRE(grp.w[g] && grp.sw[g] && grp.c[g], SPECQ_EINVAL, "w8a8: null tensor pointer");
    SPECQ_REQUIRE((layout != 0 || grp.ldw[g] >= K) && grp.ldc[g] >= N, SPECQ_EINVAL,
                  "w8a8: row strides must cover a row (lda=%lld ldw=%lld ldc=%lld)", (long long)lda,
                  (long long)grp.ldw[g], (long long)grp.ldc[g]);
    if (layout == 0) vec = std::min(vec, common_vec({(uint64_t)(uintptr_t)grp.w[g], (uint64_t)grp.ldw[g]}));
    SPECQ_REQUIRE(layout == 0 || (uintptr_t)grp.w[g] % 16 == 0, SPECQ_EINVAL, "w8a8: misaligned packed weight");
  }
  SPECQ_REQUIRE(grid_m_max == 0 || grid_m_max >= M, SPECQ_EINVAL, "w8a8: grid_m_max=%d < M=%d", grid_m_max, M);
  const int m_grid = grid_m_max > 0 ? grid_m_max : M;
  if (m_grid == 0) return SPECQ_OK;
  SPECQ_REQUIRE(layout == 0 || vec == 16, SPECQ_ENOTSUP,
                "w8a8: packed weights need 16-byte aligned activations and K %% 16 == 0");
  SPECQ_REQUIRE(layout != 2 || K <= 131072, SPECQ_ENOTSUP, "w4a8: K=%d exceeds 131072 (INT32 range of 16*sum)", K);
  W8A8Cfg cfg;
  int rc = w8a8_group_config(layout, m_grid, grp, K, block_m, block_n, num_warps, split_k, vec, plan != nullptr, &cfg);
  if (rc) return rc;
  const size_t need = cfg.ws_partials + cfg.ws_counters;
  if (static_scratch) {
    SPECQ_REQUIRE(need <= SPECQ_NOALLOC_SCRATCH_BYTES, SPECQ_ENOSPC,
                  "w8a8_packed_noalloc: this call needs %zu bytes of scratch, the static scratch holds %zu "
                  "(split_k=%d, BLOCK_M=%d); use specq_w8a8_packed with a workspace",
                  need, (size_t)SPECQ_NOALLOC_SCRATCH_BYTES, cfg.splits, cfg.mt * 16);
    if (need) {
      rc = noalloc_scratch(&workspace);
      if (rc) return rc;
      workspace_bytes = SPECQ_NOALLOC_SCRATCH_BYTES;
    }
  }
  SPECQ_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), SPECQ_ENOSPC,
                "w8a8: workspace of %zu bytes required, %zu given", need, workspace ? workspace_bytes : 0);
  rc = ensure_lds(cfg.fn, cfg.lds);
  if (rc) return rc;
  auto vec_store = [](const void* c, int64_t ldc, const float* sw) {
    return (int)(((uintptr_t)c % 8 == 0) && (ldc % 4 == 0) && ((uintptr_t)sw % 16 == 0));
  };
  W8A8Params p;
  memset(&p, 0, sizeof(p));
  p.A = a; p.lda = lda; p.W = (const int8_t*)grp.w[0]; p.ldw = grp.ldw[0]; p.sa = sa; p.sw = grp.sw[0];
  p.C = reinterpret_cast<__half*>(grp.c[0]); p.ldc = grp.ldc[0]; p.plan = plan;
  p.M = M; p.N = grp.N[0]; p.K = K; p.m_grid = m_grid;
  p.n_tiles = cfg.n_tiles; p.m_chunks = cfg.m_chunks; p.splits = cfg.splits; p.k_range = cfg.k_range;
  p.counters = need ? reinterpret_cast<int32_t*>(workspace) : nullptr;
  p.partials = need ? reinterpret_cast<int32_t*>(reinterpret_cast<char*>(workspace) + kCounterBytes) : nullptr;
  p.vec_store = vec_store(grp.c[0], grp.ldc[0], grp.sw[0]);
  diag_timeline(&p.tl, &p.tl_cap);
  p.n_grp = grp.n;
  int tile_end = 0;
  for (int g = 0; g < grp.n; ++g) {
    tile_end += ceil_div(grp.N[g], cfg.bn);
    if (g + 1 < grp.n) p.grp_tile_end[g] = tile_end;
    if (g > 0) {
      p.grp_W[g - 1] = (const int8_t*)grp.w[g]; p.grp_ldw[g - 1] = grp.ldw[g]; p.grp_sw[g - 1] = grp.sw[g];
      p.grp_C[g - 1] = reinterpret_cast<__half*>(grp.c[g]); p.grp_ldc[g - 1] = grp.ldc[g]; p.grp_N[g - 1] = grp.N[g];
      p.grp_vec_store[g - 1] = vec_store(grp.c[g], grp.ldc[g], grp.sw[g]);
    }
  }
  const int grid = cfg.family == kPlan ? cfg.plan_grid : chunked_grid(cfg.n_tiles * cfg.splits, cfg.m_chunks);
  if (static_scratch && need) {
    int n_ctr = cfg.family == kPlan ? cfg.n_counters : cfg.m_chunks * cfg.n_tiles;
    int32_t* ctr = p.counters;
    void* zargs[] = {(void*)&ctr, (void*)&n_ctr};
    const hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&zero_i32_kernel), dim3(ceil_div(n_ctr, 256)),
                                         dim3(256), zargs, 0, reinterpret_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
      set_error("w8a8_packed_noalloc: counter clear failed: %s", hipGetErrorString(e));
      return SPECQ_EIO;
    }
  }
  if (cfg.family == kPlan) {
    W8A8PlanParams pp;
    pp.p = p;
    for (int e = 0; e < kW8A8PlanRows; ++e) pp.t[e] = cfg.plan_t[e];
    return launch(cfg.fn, grid, 256, cfg.lds, reinterpret_cast<hipStream_t>(stream), &pp);
  }
  return launch(cfg.fn, grid, cfg.nw * 64, cfg.lds, reinterpret_cast<hipStream_t>(stream), &p);
}

int run_w8a8(int layout, const int8_t* a, int64_t lda, const void* w, int64_t ldw, const float* sa, const float* sw,
             void* c, int64_t ldc, int M, int N, int K, int grid_m_max, const int32_t* plan, int block_m, int block_n,
             int num_warps, int split_k, void* workspace, size_t workspace_bytes, void* stream,
             bool static_scratch = false) {
  return run_w8a8(layout, a, lda, single(w, ldw, sw, c, ldc, N), sa, M, K, grid_m_max, plan, block_m, block_n,
                  num_warps, split_k, workspace, workspace_bytes, stream, static_scratch);
}

size_t workspace_size(int layout, int m_grid, const W8A8Group& grp, int K, int block_m, int block_n, int num_warps,
                      int split_k) {
  W8A8Cfg cfg;
  size_t best = 0;
  // Size for every alignment class and mode (eager or plan) the call could resolve to.
  for (int vec : {16, 1}) {
    if ((layout != 0 || grp.n > 1) && vec != 16) continue;
    for (bool plan_mode : {false, true}) {
      if (w8a8_group_config(layout, m_grid, grp, K, block_m, block_n, num_warps, split_k, vec, plan_mode, &cfg) ==
          SPECQ_OK) {
        const size_t s = cfg.ws_partials + cfg.ws_counters;
        if (s > best) best = s;
      }
    }
  }
  clear_error();
  return best;
}

size_t workspace_size(int layout, int m_grid, int N, int K, int block_m, int block_n, int num_warps, int split_k) {
  return workspace_size(layout, m_grid, single(nullptr, 0, nullptr, nullptr, 0, N), K, block_m, block_n, num_warps,
                        split_k);
}

}  // namespace

int w8a8_attrs(int layout, int m_grid, int N, int K, int block_m, int block_n, int num_warps, int split_k,
               specq_kernel_attrs* out) {
  W8A8Cfg cfg;
  const bool plan_mode = (layout & kAttrsPlan) != 0;
  layout &= ~kAttrsPlan;
  SPECQ_REQUIRE(layout >= 0 && layout <= 2, SPECQ_EINVAL, "w8a8 attrs: layout %d", layout);
  int rc = w8a8_group_config(layout, m_grid, single(nullptr, 0, nullptr, nullptr, 0, N), K, block_m, block_n,
                             num_warps, split_k, 16, plan_mode, &cfg);
  if (rc) return rc;
  hipFuncAttributes fa;
  if (hipFuncGetAttributes(&fa, cfg.fn) != hipSuccess) return fail(SPECQ_EIO, "w8a8: hipFuncGetAttributes failed");
  // The name carries the template arguments exactly as profilers print the kernel symbol.
  const int kw = cfg.bn == 16 ? 4 : (cfg.bn == 32 ? 2 : 1), rw = cfg.bn == 128 ? 2 : 1, s = 4 / kw;
  // A plan-mode launch with automatic tiles reports its tiling for M = m_grid.
  if (cfg.family == kPlan) {
    snprintf(out->name, sizeof(out->name), "specq::w8a8_plan_kernel<%d, %d>", cfg.layout,
             cfg.fn == (cfg.layout == 0 ? w8a8_plan_fn_l0(1) : (cfg.layout == 1 ? w8a8_plan_fn_l1(1) : w8a8_plan_fn_l2(1))));
  } else if (cfg.family == kRk) {
    snprintf(out->name, sizeof(out->name), "specq::w8a8_rk_kernel<1, %d, %d, 4, %d>", rw, kw, cfg.layout);
  } else if (cfg.family == kWs) {
    const int nslot = w8a8_ws_nslot(cfg.mt, kw);
    snprintf(out->name, sizeof(out->name), "specq::w8a8_ws_kernel<%d, %d, %d, %d, %d, 4, %d>", cfg.mt, rw, kw, s,
             nslot, cfg.layout);
  } else {
    snprintf(out->name, sizeof(out->name), "specq::w8a8_kernel<%d, %d, %d>", cfg.mt, cfg.rw, cfg.vec);
  }
  out->num_regs = fa.numRegs;
  out->lds_bytes = (int)(fa.sharedSizeBytes + cfg.lds);
  out->scratch_bytes = (int)fa.localSizeBytes;
  out->threads = cfg.nw * 64;
  out->grid = cfg.family == kPlan ? cfg.plan_grid : chunked_grid(cfg.n_tiles * cfg.splits, cfg.m_chunks);
  out->block_m = cfg.mt * 16; out->block_n = cfg.bn; out->num_warps = cfg.nw; out->split_k = cfg.splits;
  return SPECQ_OK;
}

}  // namespace specq

using namespace specq;

extern "C" size_t specq_w8a8_workspace_size(int m_grid, int N, int K, int block_m, int block_n, int num_warps,
                                            int split_k) {
  return workspace_size(0, m_grid, N, K, block_m, block_n, num_warps, split_k);
}

extern "C" int specq_w8a8(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, const float* sa,
                          const float* sw, void* c, int64_t ldc, int M, int N, int K, int grid_m_max,
                          const int32_t* plan, int block_m, int block_n, int num_warps, int split_k,
                          void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return run_w8a8(0, a, lda, w, ldw, sa, sw, c, ldc, M, N, K, grid_m_max, plan, block_m, block_n, num_warps,
                  split_k, workspace, workspace_bytes, stream);
}

extern "C" size_t specq_w8a8_packed_bytes(int N, int K) {
  if (N <= 0 || K <= 0) return 0;
  return (size_t)ceil_div(N, 16) * ceil_div(K, 64) * 1024;
}

extern "C" int specq_w8a8_pack_weight(const int8_t* w, int64_t ldw, int N, int K, void* packed, void* stream) {
  clear_error();
  SPECQ_REQUIRE(w && packed, SPECQ_EINVAL, "w8a8_pack_weight: null tensor pointer");
  SPECQ_REQUIRE(N > 0 && K > 0 && ldw >= K, SPECQ_EINVAL, "w8a8_pack_weight: bad sizes N=%d K=%d ldw=%lld", N, K,
                (long long)ldw);
  SPECQ_REQUIRE((uintptr_t)packed % 16 == 0, SPECQ_EINVAL, "w8a8_pack_weight: misaligned output");
  const int64_t frags = (int64_t)ceil_div(N, 16) * ceil_div(K, 64);
  SPECQ_REQUIRE(ceil_div64(frags, 4) <= INT32_MAX, SPECQ_ENOTSUP, "w8a8_pack_weight: weight too large");
  void* args[] = {(void*)&w, (void*)&ldw, (void*)&N, (void*)&K, (void*)&packed};
  hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&w8a8_pack_kernel),
                                 dim3((unsigned)ceil_div64(frags, 4)), dim3(256), args, 0, (hipStream_t)stream);
  if (e != hipSuccess) {
    set_error("w8a8_pack_weight: hipLaunchKernel failed: %s", hipGetErrorString(e));
    return SPECQ_EIO;
  }
  return SPECQ_OK;
}

extern "C" size_t specq_w8a8_packed_workspace_size(int m_grid, int N, int K, int block_m, int block_n,
                                                   int num_warps, int split_k) {
  return workspace_size(1, m_grid, N, K, block_m, block_n, num_warps, split_k);
}

extern "C" int specq_w8a8_packed(const int8_t* a, int64_t lda, const void* w_packed, const float* sa,
                                 const float* sw, void* c, int64_t ldc, int M, int N, int K, int grid_m_max,
                                 const int32_t* plan, int block_m, int block_n, int num_warps, int split_k,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return run_w8a8(1, a, lda, w_packed, 0, sa, sw, c, ldc, M, N, K, grid_m_max, plan, block_m, block_n, num_warps,
                  split_k, workspace, workspace_bytes, stream);
}

extern "C" int specq_w8a8_packed_noalloc(const int8_t* a, int64_t lda, const void* w_packed, const float* sa,
                                         const float* sw, void* c, int64_t ldc, int M, int N, int K, int grid_m_max,
                                         const int32_t* plan, int block_m, int block_n, int num_warps, int split_k,
                                         void* stream) {
  clear_error();
  return run_w8a8(1, a, lda, w_packed, 0, sa, sw, c, ldc, M, N, K, grid_m_max, plan, block_m, block_n, num_warps,
                  split_k, nullptr, 0, stream, /*static_scratch=*/true);
}

namespace {
int make_group(int n_members, const void* const* w, const int64_t* ldw, const float* const* sw, void* const* c,
               const int64_t* ldc, const int* N, W8A8Group* grp) {
  SPECQ_REQUIRE(n_members >= 1 && n_members <= kW8A8MaxGroup, SPECQ_EINVAL,
                "w8a8_grouped: %d GEMMs (1..%d supported)", n_members, kW8A8MaxGroup);
  SPECQ_REQUIRE(N != nullptr, SPECQ_EINVAL, "w8a8_grouped: null N array");
  grp->n = n_members;
  for (int g = 0; g < n_members; ++g) {
    grp->w[g] = w ? w[g] : nullptr;
    grp->ldw[g] = ldw ? ldw[g] : 0;
    grp->sw[g] = sw ? sw[g] : nullptr;
    grp->c[g] = c ? c[g] : nullptr;
    grp->ldc[g] = ldc ? ldc[g] : 0;
    grp->N[g] = N[g];
  }
  return SPECQ_OK;
}
}  // namespace

extern "C" size_t specq_w8a8_grouped_workspace_size(int layout, int m_grid, int n_members, const int* N, int K,
                                                    int block_m, int block_n, int num_warps, int split_k) {
  W8A8Group grp;
  if (layout < 0 || layout > 2 || make_group(n_members, nullptr, nullptr, nullptr, nullptr, nullptr, N, &grp)) {
    clear_error();
    return 0;
  }
  for (int g = 0; g < n_members; ++g)
    if (N[g] <= 0) return 0;
  return workspace_size(layout, m_grid, grp, K, block_m, block_n, num_warps, split_k);
}

extern "C" int specq_w8a8_grouped(int layout, const int8_t* a, int64_t lda, const float* sa, int n_members,
                                  const void* const* w, const int64_t* ldw, const float* const* sw, void* const* c,
                                  const int64_t* ldc, const int* N, int M, int K, int grid_m_max, const int32_t* plan,
                                  int block_m, int block_n, int num_warps, int split_k, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  clear_error();
  SPECQ_REQUIRE(layout >= 0 && layout <= 2, SPECQ_EINVAL, "w8a8_grouped: weight layout %d (0, 1 or 2)", layout);
  SPECQ_REQUIRE(w && sw && c && ldc && N && (layout != 0 || ldw), SPECQ_EINVAL, "w8a8_grouped: null member array");
  W8A8Group grp;
  int rc = make_group(n_members, w, ldw, sw, c, ldc, N, &grp);
  if (rc) return rc;
  return run_w8a8(layout, a, lda, grp, sa, M, K, grid_m_max, plan, block_m, block_n, num_warps, split_k, workspace,
                  workspace_bytes, stream);
}

extern "C" int specq_set_option(const char* name, int value) {
  clear_error();
  SPECQ_REQUIRE(name != nullptr, SPECQ_EINVAL, "set_option: null name");
  if (strcmp(name, "attn_target_wgs") == 0) {
    SPECQ_REQUIRE(value >= 0 && value <= (1 << 20), SPECQ_EINVAL, "set_option: attn_target_wgs must be 0..2^20");
    g_attn_target.store(value);
    return SPECQ_OK;
  }
  if (strcmp(name, "w8a8_path") == 0) {
    SPECQ_REQUIRE(value >= 0 && value <= 3, SPECQ_EINVAL, "set_option: w8a8_path must be 0..3");
    g_w8a8_path.store(value);
    return SPECQ_OK;
  }
  if (strcmp(name, "tuned_tiles") == 0) {
    SPECQ_REQUIRE(value >= 0 && value <= 1, SPECQ_EINVAL, "set_option: tuned_tiles must be 0 or 1");
    g_tuned_tiles.store(value);
    return SPECQ_OK;
  }
  if (strcmp(name, "w4a16_path") == 0) {
    SPECQ_REQUIRE(value >= 0 && value <= 2, SPECQ_EINVAL, "set_option: w4a16_path must be 0..2");
    g_w4a16_path.store(value);
    return SPECQ_OK;
  }
  set_error("set_option: unknown option '%s'", name);
  return SPECQ_EINVAL;
}

extern "C" size_t specq_w4a8_packed_bytes(int N, int K) {
  if (N <= 0 || K <= 0) return 0;
  return (size_t)ceil_div(N, 16) * ceil_div(K, 64) * 512;
}

extern "C" int specq_w4a8_pack_weight(const void* wq, int64_t ldq, int wq_layout, int N, int K, void* packed,
                                      void* stream) {
  clear_error();
  SPECQ_REQUIRE(wq && packed, SPECQ_EINVAL, "w4a8_pack_weight: null tensor pointer");
  SPECQ_REQUIRE(wq_layout == 0 || wq_layout == 1, SPECQ_EINVAL, "w4a8_pack_weight: source layout must be 0 or 1");
  SPECQ_REQUIRE(N > 0 && K > 0 && (wq_layout == 0 ? K % 2 == 0 && ldq >= K / 2 : K % 8 == 0 && ldq >= K / 8),
                SPECQ_EINVAL, "w4a8_pack_weight: bad sizes N=%d K=%d ldq=%lld for layout %d", N, K, (long long)ldq,
                wq_layout);
  SPECQ_REQUIRE(wq_layout == 0 || (uintptr_t)wq % 4 == 0, SPECQ_EINVAL, "w4a8_pack_weight: misaligned int32 source");
  SPECQ_REQUIRE((uintptr_t)packed % 16 == 0, SPECQ_EINVAL, "w4a8_pack_weight: misaligned output");
  const int64_t frags = (int64_t)ceil_div(N, 16) * ceil_div(K, 64);
  SPECQ_REQUIRE(ceil_div64(frags, 4) <= INT32_MAX, SPECQ_ENOTSUP, "w4a8_pack_weight: weight too large");
  void* args[] = {(void*)&wq, (void*)&ldq, (void*)&wq_layout, (void*)&N, (void*)&K, (void*)&packed};
  hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&w4a8_pack_kernel),
                                 dim3((unsigned)ceil_div64(frags, 4)), dim3(256), args, 0, (hipStream_t)stream);
  if (e != hipSuccess) {
    set_error("w4a8_pack_weight: hipLaunchKernel failed: %s", hipGetErrorString(e));
    return SPECQ_EIO;
  }
  return SPECQ_OK;
}

extern "C" size_t specq_w4a8_packed_workspace_size(int m_grid, int N, int K, int block_m, int block_n,
                                                   int num_warps, int split_k) {
  return workspace_size(2, m_grid, N, K, block_m, block_n, num_warps, split_k);
}

extern "C" int specq_w4a8_packed(const int8_t* a, int64_t lda, const void* w_packed, const float* sa,
                                 const float* sw, void* c, int64_t ldc, int M, int N, int K, int grid_m_max,
                                 const int32_t* plan, int block_m, int block_n, int num_warps, int split_k,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return run_w8a8(2, a, lda, w_packed, 0, sa, sw, c, ldc, M, N, K, grid_m_max, plan, block_m, block_n, num_warps,
                  split_k, workspace, workspace_bytes, stream);
}
