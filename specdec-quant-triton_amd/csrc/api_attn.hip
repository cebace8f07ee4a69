// C ABI for the INT8 paged verification attention: validation, grid, workspace and launch.
#include <algorithm>
#include <atomic>

#include "api_common.hpp"
#include "paged_attn.hpp"

namespace specq {

// Workgroups the split length aims at (0 = the device's CUs), set through
// specq_set_option("attn_target_wgs", v); eager and plan-mode calls that are compared bit for
// bit must run with the same value.
std::atomic<int> g_attn_target{0};

const void* attn_plan_fn_d64(int rb_max, int fp32);   // attn_plan_d64.hip
const void* attn_plan_fn_d128(int rb_max, int fp32);  // attn_plan_d128.hip

namespace {

template <int D>
const void* attn_fn_d(int rb, int fp32) {
  switch (rb * 2 + fp32) {
    case 2: return reinterpret_cast<const void*>(&paged_attn_kernel<D, 1, _Float16>);
    case 3: return reinterpret_cast<const void*>(&paged_attn_kernel<D, 1, float>);
    case 4: return reinterpret_cast<const void*>(&paged_attn_kernel<D, 2, _Float16>);
    case 5: return reinterpret_cast<const void*>(&paged_attn_kernel<D, 2, float>);
    case 6: return reinterpret_cast<const void*>(&paged_attn_kernel<D, 3, _Float16>);
    case 7: return reinterpret_cast<const void*>(&paged_attn_kernel<D, 3, float>);
    case 8: return reinterpret_cast<const void*>(&paged_attn_kernel<D, 4, _Float16>);
    case 9: return reinterpret_cast<const void*>(&paged_attn_kernel<D, 4, float>);
  }
  return nullptr;
}

const void* attn_fn(int D, int rb, int fp32) {
  if (D == 128) return attn_fn_d<128>(rb, fp32);
  if (D == 64) return attn_fn_d<64>(rb, fp32);
  return nullptr;
}

// grid.x: the splits of a block table of max_pages * PAGE tokens when at least `pairs_min`
// (sequence, KV head) pairs are active (fewer pairs never means fewer splits).
int n_splits_for(int max_pages, int PAGE, int pairs_min, int target) {
  const int cap = max_pages * PAGE;
  const int per = kAttnUnit * attn_split_units(cap, pairs_min, target);
  return std::max(1, ceil_div(cap, per));
}

}  // namespace

// `variant` is the head dim, | kAttrsScaleFp32 for fp32 K/V scales.
int attn_attrs(int variant, int rows, specq_kernel_attrs* out) {
  const bool fp32 = (variant & kAttrsScaleFp32) != 0;
  const int D = variant & ~kAttrsScaleFp32;
  SPECQ_REQUIRE(rows >= 1 && rows <= 64, SPECQ_ENOTSUP, "paged_attn: %d packed rows (1..64 supported)", rows);
  const int rb = ceil_div(rows, 16);
  const void* fn = attn_fn(D, rb, fp32 ? 1 : 0);
  SPECQ_REQUIRE(fn != nullptr, SPECQ_ENOTSUP, "paged_attn: head_dim %d not supported", D);
  hipFuncAttributes fa;
  if (hipFuncGetAttributes(&fa, fn) != hipSuccess) return fail(SPECQ_EIO, "paged_attn: hipFuncGetAttributes failed");
  // The name carries the template arguments exactly as profilers print the kernel symbol.
  snprintf(out->name, sizeof(out->name), "specq::paged_attn_kernel<%d, %d, %s>", D, rb, fp32 ? "float" : "_Float16");
  out->num_regs = fa.numRegs;
  out->lds_bytes = (int)fa.sharedSizeBytes;
  out->scratch_bytes = (int)fa.localSizeBytes;
  out->threads = kAttnThreads;
  out->block_m = rb * 16;
  return SPECQ_OK;
}

}  // namespace specq

using namespace specq;

extern "C" size_t specq_paged_attn_workspace_size(int B_grid, int H, int H_KV, int ql_grid, int QPP, int max_pages,
                                                  int PAGE) {
  if (B_grid <= 0 || H_KV <= 0 || H % H_KV != 0 || QPP <= 0 || ql_grid <= 0 || max_pages <= 0 || PAGE <= 0) return 0;
  const int G = H / H_KV;
  const int rows = ceil_div(QPP * G, 16) * 16;
  const int n_qc = ceil_div(ql_grid, QPP);
  const int64_t progs = (int64_t)B_grid * H_KV * n_qc;
  if ((int64_t)max_pages * PAGE > kAttnMaxTokens) return 0;
  // Plan-mode bound: at least one active sequence.
  const int tgt = g_attn_target.load();
  const int ns = n_splits_for(max_pages, PAGE, H_KV, tgt > 0 ? tgt : device_cus());
  if (ns <= 1) return 0;
  // Sized for D = 128 (the largest supported head dimension).
  const size_t part = (size_t)progs * ns * rows * (128 + 2) * 4;
  return kCounterBytes + align_up(part, 256);
}

extern "C" int specq_paged_attn(const void* q, int64_t s_qb, int64_t s_qt, int64_t s_qh, const int8_t* kc,
                                const int8_t* vc, int64_t s_kp, int64_t s_ko, int64_t s_kh, const void* ks,
                                const void* vs, int64_t s_sp, int64_t s_so, int64_t s_sh, int scale_fp32,
                                const int32_t* block_tbl, int64_t s_bt, int max_pages, int n_pages,
                                const int32_t* ctx_len,
                                void* out, int64_t s_ob, int64_t s_ot, int64_t s_oh, int B_grid, int n_seqs,
                                int q_len, int ql_grid, int H, int H_KV, int D, int PAGE, int QPP, float sm_scale,
                                const int32_t* plan, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  SPECQ_REQUIRE(q && kc && vc && ks && vs && block_tbl && ctx_len && out, SPECQ_EINVAL,
                "paged_attn: null tensor pointer");
  SPECQ_REQUIRE(B_grid >= 0 && ql_grid > 0 && H > 0 && H_KV > 0 && H % H_KV == 0, SPECQ_EINVAL,
                "paged_attn: bad sizes B=%d ql=%d H=%d H_KV=%d", B_grid, ql_grid, H, H_KV);
  SPECQ_REQUIRE(D == 64 || D == 128, SPECQ_ENOTSUP, "paged_attn: head_dim %d (64 or 128 supported)", D);
  SPECQ_REQUIRE(PAGE > 0 && PAGE % 16 == 0, SPECQ_ENOTSUP, "paged_attn: PAGE=%d must be a multiple of 16", PAGE);
  SPECQ_REQUIRE(max_pages > 0, SPECQ_EINVAL, "paged_attn: empty block table");
  SPECQ_REQUIRE(n_pages > 0, SPECQ_EINVAL, "paged_attn: empty K/V pool (n_pages=%d)", n_pages);
  SPECQ_REQUIRE((int64_t)max_pages * PAGE <= kAttnMaxTokens, SPECQ_ENOTSUP,
                "paged_attn: block table of %lld tokens exceeds %lld", (long long)max_pages * PAGE,
                (long long)kAttnMaxTokens);
  SPECQ_REQUIRE(QPP > 0, SPECQ_EINVAL, "paged_attn: QPP=%d", QPP);
  const int G = H / H_KV;
  SPECQ_REQUIRE(QPP * G <= 64, SPECQ_ENOTSUP, "paged_attn: QPP*G=%d packed rows exceed 64", QPP * G);
  if (plan == nullptr) {
    SPECQ_REQUIRE(n_seqs >= 0 && n_seqs <= B_grid && q_len >= 0 && q_len <= ql_grid, SPECQ_EINVAL,
                  "paged_attn: n_seqs=%d q_len=%d outside the grid (%d, %d)", n_seqs, q_len, B_grid, ql_grid);
  }
  SPECQ_REQUIRE((uintptr_t)q % 16 == 0 && s_qb % 8 == 0 && s_qt % 8 == 0 && s_qh % 8 == 0, SPECQ_ENOTSUP,
                "paged_attn: q rows must be 16-byte aligned");
  SPECQ_REQUIRE((uintptr_t)out % 16 == 0 && s_ob % 8 == 0 && s_ot % 8 == 0 && s_oh % 8 == 0, SPECQ_ENOTSUP,
                "paged_attn: out rows must be 16-byte aligned");
  SPECQ_REQUIRE((uintptr_t)kc % 16 == 0 && (uintptr_t)vc % 16 == 0 && s_kp % 16 == 0 && s_ko % 16 == 0 &&
                    s_kh % 16 == 0,
                SPECQ_ENOTSUP, "paged_attn: K/V cache rows must be 16-byte aligned");
  SPECQ_REQUIRE(s_ko > 0 && 16 * s_ko + D < ((int64_t)1 << 31), SPECQ_ENOTSUP,
                "paged_attn: token stride %lld of the K/V cache outside (0, 2^27)", (long long)s_ko);
  if (B_grid == 0) return SPECQ_OK;
  const int rb = ceil_div(QPP * G, 16);
  // Plan mode with more than one row block runs the launch that sizes its programs to the
  // active q_len on the device (the rows of a program whose queries are inactive do nothing).
  const void* fn = plan != nullptr && rb > 1
                       ? (D == 128 ? attn_plan_fn_d128(rb, scale_fp32 ? 1 : 0) : attn_plan_fn_d64(rb, scale_fp32 ? 1 : 0))
                       : attn_fn(D, rb, scale_fp32 ? 1 : 0);
  SPECQ_REQUIRE(fn != nullptr, SPECQ_ENOTSUP, "paged_attn: no kernel for D=%d rows=%d", D, QPP * G);
  const int n_qc = ceil_div(plan ? ql_grid : q_len, QPP);
  if (n_qc == 0) return SPECQ_OK;
  const int target = g_attn_target.load() > 0 ? g_attn_target.load() : device_cus();
  // Eager calls know the active sequences; a plan may activate as few as one.
  const int ns = n_splits_for(max_pages, PAGE, (plan ? 1 : std::max(n_seqs, 1)) * H_KV, target);
  const int64_t progs = (int64_t)B_grid * H_KV * n_qc;
  const int rows = rb * 16;
  size_t need = 0;
  if (ns > 1) {
    SPECQ_REQUIRE(progs <= kMaxCounters, SPECQ_ENOTSUP, "paged_attn: %lld programs exceed the counter region",
                  (long long)progs);
    need = kCounterBytes + align_up((size_t)progs * ns * rows * (D + 2) * 4, 256);
  }
  SPECQ_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), SPECQ_ENOSPC,
                "paged_attn: workspace of %zu bytes required, %zu given", need, workspace ? workspace_bytes : 0);
  // One-dimensional grid of program x split (the kernel derives both from the active count):
  // the exact count for an eager call, the most any active count needs in plan mode.
  int64_t wgs = (int64_t)(plan ? B_grid : n_seqs) * H_KV * n_qc * ns;
  if (plan) {
    wgs = 0;
    for (int s = 1; s <= B_grid; ++s)
      wgs = std::max(wgs, (int64_t)s * H_KV * n_qc * n_splits_for(max_pages, PAGE, s * H_KV, target));
  }
  if (wgs == 0) return SPECQ_OK;
  SPECQ_REQUIRE(wgs <= INT32_MAX, SPECQ_ENOTSUP, "paged_attn: grid too large");
  AttnParams p;
  p.q = (const _Float16*)q; p.s_qb = s_qb; p.s_qt = s_qt; p.s_qh = s_qh;
  p.kc = kc; p.vc = vc; p.s_kp = s_kp; p.s_ko = s_ko; p.s_kh = s_kh;
  p.ks = ks; p.vs = vs; p.s_sp = s_sp; p.s_so = s_so; p.s_sh = s_sh;
  p.bt = block_tbl; p.s_bt = s_bt; p.max_pages = max_pages; p.n_pages = n_pages; p.ctx_len = ctx_len;
  p.out = (_Float16*)out; p.s_ob = s_ob; p.s_ot = s_ot; p.s_oh = s_oh;
  p.plan = plan; p.B_grid = B_grid; p.n_seqs = plan ? B_grid : n_seqs; p.q_len = plan ? ql_grid : q_len;
  p.ql_grid = ql_grid; p.G = G; p.QPP = QPP; p.n_qc = n_qc; p.H_KV = H_KV; p.PAGE = PAGE; p.n_splits = ns;
  p.target_wgs = target;
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  p.counters = need ? (int32_t*)workspace : nullptr;
  p.part = need ? (float*)((char*)workspace + kCounterBytes) : nullptr;
  diag_timeline(&p.tl, &p.tl_cap);
  void* args[] = {&p};
  hipError_t e = hipLaunchKernel(fn, dim3((unsigned)wgs), dim3(kAttnThreads), args, 0, (hipStream_t)stream);
  if (e != hipSuccess) {
    set_error("paged_attn: hipLaunchKernel failed: %s", hipGetErrorString(e));
    return SPECQ_EIO;
  }
  return SPECQ_OK;
}
