// Paged INT8 KV-cache append and its C ABI.
//
// Writes the q_len new tokens of every sequence into the paged INT8 cache that the
// verification attention reads: token i of sequence b sits at position
// pos = ctx_len[b] - q_len + i (ctx_len counts the new tokens, as the attention's does,
// kernels.py:173), i.e. in page block_tbl[b, pos / PAGE], slot pos % PAGE.  Each (token, KV
// head) row of D values is quantised symmetrically, as the reference builds its cache
// (kernels.py:280-284):
//   s = max(amax_d |x[d]|, 1e-8) / 127 (fp32, IEEE division),
//   q[d] = clamp(rne(x[d] / s), -127, 127),
// and s is stored as fp16 (RNE) or fp32.
//
// One workgroup per (sequence, new token): its 2 * H_KV rows (K rows, then V rows) are spread
// over groups of LPR = D / 8 lanes, each lane holding 8 values (one 16-byte load), so the row
// amax is a shuffle reduction inside the lane group and the quantised row leaves as one
// 8-byte store per lane.  The kernel is HBM-bound: 2 * D bytes read and D + scale bytes
// written per row.  Sequences or tokens beyond the active (n_seqs, q_len) exit (plan mode
// reads them from the device), and rows whose position or page falls outside the cache are
// skipped rather than written.
#include "api_common.hpp"
#include "common.hpp"

namespace specq {

struct KvAppendParams {
  const _Float16* k; const _Float16* v; int64_t s_nb, s_nt, s_nh;  // new K/V [B, ql, H_KV, D]
  int8_t* kc; int8_t* vc; int64_t s_kp, s_ko, s_kh;               // caches [pages, PAGE, H_KV, D]
  void* ks; void* vs; int64_t s_sp, s_so, s_sh;                   // scales [pages, PAGE, H_KV]
  const int32_t* bt; int64_t s_bt; int max_pages, n_pages;
  const int32_t* ctx_len;
  const int32_t* plan;
  int n_seqs, q_len, ql_grid, B_grid, H_KV, PAGE;
};

template <int LPR, bool SF32>
__global__ __launch_bounds__(256) void kv_append_kernel(KvAppendParams p) {
  constexpr int RPP = 256 / LPR;  // rows per pass
  const int b = blockIdx.x / p.ql_grid, i = blockIdx.x % p.ql_grid;
  const int t = threadIdx.x, grp = t / LPR, l = t % LPR;
  auto row_src = [&](int row) {
    const bool is_v = row >= p.H_KV;
    const int h = is_v ? row - p.H_KV : row;
    return (is_v ? p.v : p.k) + (int64_t)b * p.s_nb + (int64_t)i * p.s_nt + (int64_t)h * p.s_nh + 8 * l;
  };
  // The first pass's new K/V values and the context length depend on neither the plan nor
  // the block table (every (b, i) of the grid lies inside the new K/V tensor and ctx_len), so
  // their loads go out together with the plan's instead of after it.
  v8h x_first = {};
  if (grp < 2 * p.H_KV) x_first = *reinterpret_cast<const v8h*>(row_src(grp));
  const int L = p.ctx_len[b];
  int nb = p.n_seqs, ql = p.q_len;
  if (p.plan != nullptr) {
    nb = min(max(p.plan[0], 0), p.B_grid);
    ql = min(max(p.plan[1], 0), p.ql_grid);
  }
  nb = uniform(nb);
  ql = uniform(ql);
  if (b >= nb || i >= ql) return;
  const int pos = uniform(L - ql + i);
  if (pos < 0 || pos / p.PAGE >= p.max_pages) return;
  const int page = uniform(p.bt[(int64_t)b * p.s_bt + pos / p.PAGE]);
  if (page < 0 || page >= p.n_pages) return;
  const int slot = pos % p.PAGE;

  for (int row = grp; row < 2 * p.H_KV; row += RPP) {
    const bool is_v = row >= p.H_KV;
    const int h = is_v ? row - p.H_KV : row;
    const v8h x = row == grp ? x_first : *reinterpret_cast<const v8h*>(row_src(row));
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf((float)x[j]));
#pragma unroll
    for (int o = LPR / 2; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    const float s = fmaxf(amax, 1e-8f) / 127.0f;
    int w[2] = {0, 0};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float q = rintf((float)x[j] / s);
      q = fminf(fmaxf(q, -127.f), 127.f);
      w[j >> 2] |= ((int)q & 0xff) << (8 * (j & 3));
    }
    int8_t* dst = (is_v ? p.vc : p.kc) + (int64_t)page * p.s_kp + (int64_t)slot * p.s_ko + (int64_t)h * p.s_kh;
    *reinterpret_cast<v2i*>(dst + 8 * l) = v2i{w[0], w[1]};
    if (l == 0) {
      const int64_t so = (int64_t)page * p.s_sp + (int64_t)slot * p.s_so + (int64_t)h * p.s_sh;
      void* sp = is_v ? p.vs : p.ks;
      if constexpr (SF32) static_cast<float*>(sp)[so] = s;
      else static_cast<_Float16*>(sp)[so] = (_Float16)s;
    }
  }
}

template <bool SF32>
static const void* kv_append_fn(int D) {
  switch (D) {
    case 64: return reinterpret_cast<const void*>(&kv_append_kernel<8, SF32>);
    case 128: return reinterpret_cast<const void*>(&kv_append_kernel<16, SF32>);
    case 256: return reinterpret_cast<const void*>(&kv_append_kernel<32, SF32>);
  }
  return nullptr;
}

}  // namespace specq

using namespace specq;

extern "C" int specq_kv_append_int8(const void* k_new, const void* v_new, int64_t s_nb, int64_t s_nt, int64_t s_nh,
                                    int8_t* kc, int8_t* vc, int64_t s_kp, int64_t s_ko, int64_t s_kh, void* ks,
                                    void* vs, int64_t s_sp, int64_t s_so, int64_t s_sh, int scale_fp32,
                                    const int32_t* block_tbl, int64_t s_bt, int max_pages, int n_pages,
                                    const int32_t* ctx_len, int B_grid, int n_seqs, int q_len, int ql_grid,
                                    int H_KV, int D, int PAGE, const int32_t* plan, void* stream) {
  clear_error();
  SPECQ_REQUIRE(k_new && v_new && kc && vc && ks && vs && block_tbl && ctx_len, SPECQ_EINVAL,
                "kv_append_int8: null tensor pointer");
  SPECQ_REQUIRE(B_grid >= 0 && ql_grid >= 0 && n_seqs >= 0 && n_seqs <= B_grid && q_len >= 0 && q_len <= ql_grid,
                SPECQ_EINVAL, "kv_append_int8: need 0 <= n_seqs <= B_grid and 0 <= q_len <= ql_grid");
  SPECQ_REQUIRE(H_KV > 0 && PAGE > 0 && max_pages > 0 && n_pages > 0, SPECQ_EINVAL, "kv_append_int8: bad sizes");
  const void* fn = scale_fp32 ? kv_append_fn<true>(D) : kv_append_fn<false>(D);
  SPECQ_REQUIRE(fn != nullptr, SPECQ_ENOTSUP, "kv_append_int8: head_dim %d must be 64, 128 or 256", D);
  SPECQ_REQUIRE((uintptr_t)k_new % 16 == 0 && (uintptr_t)v_new % 16 == 0 && s_nb % 8 == 0 && s_nt % 8 == 0 &&
                    s_nh % 8 == 0,
                SPECQ_ENOTSUP, "kv_append_int8: new K/V rows must be 16-byte aligned");
  SPECQ_REQUIRE((uintptr_t)kc % 8 == 0 && (uintptr_t)vc % 8 == 0 && s_kp % 8 == 0 && s_ko % 8 == 0 && s_kh % 8 == 0,
                SPECQ_ENOTSUP, "kv_append_int8: cache rows must be 8-byte aligned");
  SPECQ_REQUIRE(s_kh >= D && s_nh >= D && s_bt >= max_pages, SPECQ_EINVAL, "kv_append_int8: bad strides");
  if (B_grid == 0 || ql_grid == 0) return SPECQ_OK;
  SPECQ_REQUIRE((int64_t)B_grid * ql_grid <= 0x7fffffff, SPECQ_EINVAL, "kv_append_int8: grid too large");
  KvAppendParams p = {};
  p.k = (const _Float16*)k_new; p.v = (const _Float16*)v_new; p.s_nb = s_nb; p.s_nt = s_nt; p.s_nh = s_nh;
  p.kc = kc; p.vc = vc; p.s_kp = s_kp; p.s_ko = s_ko; p.s_kh = s_kh;
  p.ks = ks; p.vs = vs; p.s_sp = s_sp; p.s_so = s_so; p.s_sh = s_sh;
  p.bt = block_tbl; p.s_bt = s_bt; p.max_pages = max_pages; p.n_pages = n_pages;
  p.ctx_len = ctx_len; p.plan = plan;
  p.n_seqs = n_seqs; p.q_len = q_len; p.ql_grid = ql_grid; p.B_grid = B_grid; p.H_KV = H_KV; p.PAGE = PAGE;
  return launch(fn, B_grid * ql_grid, 256, 0, (hipStream_t)stream, &p);
}
