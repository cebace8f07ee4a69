/*
 * specq.h -- C ABI of libspecq.so, the gfx950 (MI355X) quantized speculative-decoding
 * verification kernels.
 *
 * Each entry point replaces one launcher of the reference's kernels.py and takes plain
 * device pointers, element strides and sizes (no framework types).  All launches are
 * asynchronous on the caller's HIP stream (`stream` is a hipStream_t, NULL = the null
 * stream); no entry point allocates, frees or synchronizes, so every one of them may be
 * recorded into a hipGraph.  Strides are in elements of the tensor's own dtype; the
 * innermost dimension of every tensor must be contiguous (stride 1).
 *
 * Plan mode (the reference's USE_PLAN, kernels.py:14-17): when `plan` is non-NULL the
 * active problem size is read on the device from that int32 buffer at kernel run time and
 * the grid is sized from the host-side maxima, so one captured graph serves every shape.
 * Plan values are clamped to the maxima the grid was sized for.  Inactive rows/sequences/
 * query slots are never written.
 *
 * Workspaces: kernels that split a reduction across workgroups need device scratch of at
 * least the size returned by the matching *_workspace_size() call.  Every workspace starts
 * with a fixed 256 KiB counter region (SPECQ_WORKSPACE_COUNTER_BYTES) followed by scratch.
 * The counter region must be zero-filled once when the workspace is created; every kernel
 * returns the counters it used to zero, so one workspace can serve any sequence of calls,
 * of any kernel and size, issued in stream order.  Calls that may run concurrently
 * (different streams) must not share a workspace.
 *
 * Return codes: 0 on success, otherwise a negative errno-style code; the message is
 * available from specq_last_error() (per calling thread).  Arguments are validated before
 * any HIP call is made.
 */
#ifndef SPECQ_H
#define SPECQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPECQ_OK 0
#define SPECQ_EIO (-5)       /* HIP launch/runtime error */
#define SPECQ_EINVAL (-22)   /* invalid argument (null pointer, bad size or stride) */
#define SPECQ_ENOSPC (-28)   /* workspace missing or too small */
#define SPECQ_ENOTSUP (-95)  /* valid but unsupported configuration (tile, head_dim, ...) */

#define SPECQ_WORKSPACE_COUNTER_BYTES (256 * 1024)

/* Library ABI version (major * 100 + minor). */
int specq_version(void);

/* Message describing the last error raised on this thread ("" if none). */
const char* specq_last_error(void);

/* ---------------------------------------------------------------------------------------
 * W8A8 GEMM: C[m, n] = fp16( (float(sum_k A[m,k] * W[n,k]) * sa[m]) * sw[n] ),  m < M, n < N
 * Replaces w8a8_matmul (kernels.py:71-86) and _w8a8_kernel (kernels.py:27-55).
 *   a        int8 [M, K], row stride lda          (a_q)
 *   w        int8 [N, K], row stride ldw          (w_q, "W^T" addressing, kernels.py:43)
 *   sa       fp32 [M] per-token scale;  sw  fp32 [N] per-channel scale
 *   c        fp16 [M, N], row stride ldc
 *   grid_m_max  rows the grid is sized for (>= M); 0 means M.  The reference's grid_m_max.
 *   plan     NULL, or device int32*: plan[0] = active M (kernels.py:35-38)
 *   block_m  token rows per workgroup: a multiple of 16, at most 304 (the reference's
 *            BLOCK_M; 16/32/64/128 are its values); 0 = automatic.  Eager calls then take
 *            the token-tile depth, channel block and split count from a cost model fitted to
 *            measured latencies; calls with a plan and block_n = split_k = 0 launch a kernel
 *            that holds a menu of tilings and runs, on the device, the one the model chose
 *            for each 16 rows of the active M (plan[0]).  Every tiling gives the same result.
 *   block_n  output channels per workgroup: 16, 32, 64 or 128; 0 = auto (chosen with split_k
 *            from M, N and K by a cost model fitted to measured latencies).  (BLOCK_N)
 *   num_warps  waves per workgroup of the byte-granular fallback kernel (unaligned operands):
 *            1, 2 or 4 (8 is taken as 4); 0 = 4.  The streaming kernels always run 4 waves.
 *   split_k  workgroups splitting K; 0 = auto.  The INT32 result does not depend on it.
 * ------------------------------------------------------------------------------------- */
size_t specq_w8a8_workspace_size(int m_grid, int N, int K, int block_m, int block_n,
                                 int num_warps, int split_k);
int specq_w8a8(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw,
               const float* sa, const float* sw, void* c, int64_t ldc,
               int M, int N, int K, int grid_m_max, const int32_t* plan,
               int block_m, int block_n, int num_warps, int split_k,
               void* workspace, size_t workspace_bytes, void* stream);

/* W8A8 with the weight pre-packed once into MFMA fragments (the layout production inference
 * stacks "pre-shuffle" weights into at load time), stored K-step-major:
 * packed[s][t][l*16 + b] = w[16t + l%16][64s + 16*(l/16) + b] for 64-byte K step s, 16-row
 * tile t (ceil(N/16) tiles per step), lane l, byte b, zero-padded to whole tiles;
 * specq_w8a8_packed_bytes() bytes.  Each 1 KB fragment is one MFMA operand, and the
 * workgroups running at one time read one compact window of the buffer.  Results are
 * bit-identical to specq_w8a8 on the unpacked weight.  No reference counterpart:
 * w8a8_matmul (kernels.py:71-86) takes the row-major weight only. */
size_t specq_w8a8_packed_bytes(int N, int K);
int specq_w8a8_pack_weight(const int8_t* w, int64_t ldw, int N, int K, void* packed, void* stream);
size_t specq_w8a8_packed_workspace_size(int m_grid, int N, int K, int block_m, int block_n,
                                        int num_warps, int split_k);
int specq_w8a8_packed(const int8_t* a, int64_t lda, const void* w_packed,
                      const float* sa, const float* sw, void* c, int64_t ldc,
                      int M, int N, int K, int grid_m_max, const int32_t* plan,
                      int block_m, int block_n, int num_warps, int split_k,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Grouped W8A8: up to 4 GEMMs that share one activation (a, sa, M, K) -- q, k and v, or gate and
 * up -- in one launch, each with its own weight, channel scale, output and N:
 *   C_g[m, n] = fp16( (float(sum_k A[m,k] * W_g[n,k]) * sa[m]) * sw_g[n] ),  n < N[g]
 * Results are bit-identical to one specq_w8a8 / specq_w8a8_packed / specq_w4a8_packed call per
 * member.  The tiles are those of one GEMM of width sum(N), so the launch costs what the fused
 * weight of bench_matmul.py:16 (qkv 6144, gate_up 28672) costs, while the weights and outputs
 * stay separate tensors as in a model's layers.  No reference counterpart (the reference fuses
 * the weights instead).
 *   layout   0 row-major int8 weights (ldw[g] row strides), 1 packed int8 (specq_w8a8_pack_weight),
 *            2 packed INT4 (specq_w4a8_pack_weight); ldw may be NULL unless layout is 0
 *   w, sw, c, ldc, N  arrays of n_members entries (host memory)
 *   Activations must have 16-byte aligned rows and K % 16 == 0.  Other arguments as specq_w8a8. */
size_t specq_w8a8_grouped_workspace_size(int layout, int m_grid, int n_members, const int* N, int K,
                                         int block_m, int block_n, int num_warps, int split_k);
int specq_w8a8_grouped(int layout, const int8_t* a, int64_t lda, const float* sa, int n_members,
                       const void* const* w, const int64_t* ldw, const float* const* sw,
                       void* const* c, const int64_t* ldc, const int* N,
                       int M, int K, int grid_m_max, const int32_t* plan,
                       int block_m, int block_n, int num_warps, int split_k,
                       void* workspace, size_t workspace_bytes, void* stream);

/* W8A8 on packed weights without a workspace argument: the same computation and tiles as
 * specq_w8a8_packed (bit-identical results), with the split-K counters and INT32 partial tiles
 * held in a static device array of SPECQ_NOALLOC_SCRATCH_BYTES bytes that each GPU keeps for the
 * life of the process.  No reference counterpart: it is for callers that cannot allocate device
 * memory (code under graph capture, serving loops that forbid allocation).  It allocates and
 * frees nothing.  A call whose tiles need more scratch than the array holds returns
 * SPECQ_ENOSPC before any launch (every config-1 shape at M <= 300 with the automatic tile fits).
 * The counters a call uses are zeroed by a fill kernel on `stream` before the GEMM.  Every call
 * on a GPU shares that GPU's array, so calls that may overlap on one GPU (different streams)
 * race and must not be issued concurrently. */
#define SPECQ_NOALLOC_SCRATCH_BYTES (32u * 1024u * 1024u)
int specq_w8a8_packed_noalloc(const int8_t* a, int64_t lda, const void* w_packed,
                              const float* sa, const float* sw, void* c, int64_t ldc,
                              int M, int N, int K, int grid_m_max, const int32_t* plan,
                              int block_m, int block_n, int num_warps, int split_k, void* stream);

/* ---------------------------------------------------------------------------------------
 * W4A8 GEMM: C[m, n] = fp16( (float(sum_k A[m,k] * q[n,k]) * sa[m]) * sw[n] ) with q the
 * signed INT4 weight in [-8, 7] and a per-channel fp32 scale sw, so the INT4 weights run on
 * the INT8 MFMA path and their scale moves to the W8A8 epilogue (the reference's
 * recommendation for INT4, REPORT.md:156; it has no W4A8 kernel).  The INT32 sums are exact,
 * so results are bit-identical to specq_w8a8 on the unpacked weight q.
 *   The weight is packed once at load from the reference INT4 packing (wq_layout 0: uint8
 *   [N, K/2], byte j of a row holding k = j in its low and k = j + K/2 in its high nibble,
 *   kernels.py:143-145; or wq_layout 1: int32 [N, K/8], nibble i of word j holding k = 8j + i;
 *   nibbles carry offset 8) into 512-byte fragments stored K-step-major: fragment (s, t) of
 *   64-wide K step s and 16-row tile t at (s * ceil(N/16) + t) * 512; lane l's dword d, byte i
 *   holds the two's-complement nibbles of w[16t + l%16][64s + 16*(l/16) + 8d + i] (low) and
 *   [... + 8d + 4 + i] (high), zero-padded.  specq_w4a8_packed_bytes() bytes.
 *   Activations as specq_w8a8_packed (16-byte aligned rows, K % 16 == 0); K <= 131072.
 *   Tiles, plan mode and workspace as specq_w8a8_packed.
 * ------------------------------------------------------------------------------------- */
size_t specq_w4a8_packed_bytes(int N, int K);
int specq_w4a8_pack_weight(const void* wq, int64_t ldq, int wq_layout, int N, int K, void* packed,
                           void* stream);
size_t specq_w4a8_packed_workspace_size(int m_grid, int N, int K, int block_m, int block_n,
                                        int num_warps, int split_k);
int specq_w4a8_packed(const int8_t* a, int64_t lda, const void* w_packed,
                      const float* sa, const float* sw, void* c, int64_t ldc,
                      int M, int N, int K, int grid_m_max, const int32_t* plan,
                      int block_m, int block_n, int num_warps, int split_k,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Tuning options.  "w8a8_path": W8A8 kernel family, 0 = automatic, 1 = direct-activation
 * streaming kernel (16-row token tiles), 2 = streaming with LDS-staged activations (tiles of
 * 32 rows or more; 16-row requests use family 1), 3 = byte-granular register kernel
 * (row-major weights only).  Every family computes the same INT32 sums, so results do not
 * change.  "w4a16_path": W4A16 kernel family, 0 = automatic (LDS-staged activations), 1 =
 * register-stream kernel for token tiles of up to 32 rows, 2 = LDS-staged activations.  Both sum in the
 * same fp32 order, so results do not change either.  "attn_target_wgs": the workgroup count
 * the paged attention's split length aims at (0 = the device's CU count); results depend on
 * the split length, so calls compared bit for bit must use the same value.  "tuned_tiles":
 * 1 (default) = eager GEMM calls with automatic tiles on the Llama-3-8B launch shapes run the
 * tile measured fastest for their 16-row step of M (a table built on a 256-CU MI355X), 0 = the
 * cost models only; W8A8 results do not change, W4A16 results do not change within a weight
 * layout's K order. */
int specq_set_option(const char* name, int value);

/* ---------------------------------------------------------------------------------------
 * W4A16 GEMM: C[m, n] = fp16( sum_k a[m,k] * fp16(fp16(q[n,k]) * sc[n, k/group]) )
 * with q the signed int4 weight in [-8, 7] stored as an unsigned nibble with offset 8.
 * Replaces w4a16_matmul (kernels.py:150-166) and _w4a16_kernel (kernels.py:94-135).
 *   a        fp16 [M, K], row stride lda
 *   wq       packed weights, row stride ldq in elements of the layout's storage type:
 *            layout 0 (reference, kernels.py:89-92, 143-145): uint8 [N, K/2]; byte j of a row
 *              holds k = j in its low nibble and k = j + K/2 in its high nibble.
 *            layout 1: int32 [N, K/8]; nibble i (bits 4i..4i+3) of word j holds k = 8j + i.
 *            layout 2: the output of specq_w4a16_pack_weight (ldq is ignored).
 *   sc       fp16 [N, K/group] group scales, row stride ld_sc
 *   group    K group size: a power of two, a multiple of 32 (layouts 1, 2) or 16 (layout 0),
 *            dividing K.  K must be a multiple of 128.
 *   block_m  token rows per tile, a multiple of 16 up to 256 (tiles deeper than 144 rows
 *            run as equal chunks of at most 144 rows; 0 = automatic; with a plan
 *            and block_n = 0 the launch holds a menu of tilings and runs, for each 16 rows
 *            of the active M, the one the eager cost model picks there);
 *   block_n  64 or 128 channels per workgroup (0 = automatic); num_warps is ignored (the
 *            LDS-staged kernels run 8 waves, the register-stream family 4).
 *   Other arguments as specq_w8a8.  The fp32 accumulation order depends only on (N, K),
 *   split_k (0 = automatic, chosen from N and K) and whether the layout is the reference one:
 *   split s takes a contiguous range of 128-wide K blocks and sums the blocks at even and at
 *   odd local index as two streams, each from zero in block order, then adds them (even +
 *   odd); the splits are added in split order.  A block is k in [128b, 128b + 128) for
 *   layouts 1 and 2 and the two runs [64b, 64b + 64) and K/2 + [64b, 64b + 64) for layout 0.
 *   It never depends on M, block_m, block_n or the plan, so those give bit-identical results,
 *   and so do layouts 1 and 2.
 * ------------------------------------------------------------------------------------- */
size_t specq_w4a16_workspace_size(int m_grid, int N, int K, int block_m, int block_n,
                                  int num_warps, int split_k);
int specq_w4a16(const void* a, int64_t lda, const void* wq, int64_t ldq, int wq_layout,
                const void* sc, int64_t ld_sc, void* c, int64_t ldc,
                int M, int N, int K, int group, int grid_m_max, const int32_t* plan,
                int block_m, int block_n, int num_warps, int split_k,
                void* workspace, size_t workspace_bytes, void* stream);

/* Grouped W4A16: up to 4 GEMMs that share one fp16 activation (a, M, K, group) -- q, k and v,
 * or gate and up -- in one launch, each with its own packed weight, group scales, output and N:
 *   C_g[m, n] = fp16( sum_k a[m,k] * fp16(fp16(q_g[n,k]) * sc_g[n, k/group]) ),  n < N[g]
 * Results are bit-identical to one specq_w4a16 call per member with the same split_k: every
 * member keeps the split count its own call would use (split_k, or the automatic count of its
 * N and K), and W4A16 results do not depend on the tiles.  When the members' automatic counts
 * differ the members run as one launch each, in order on `stream`.  Otherwise the tiles are
 * those of one GEMM of width sum(N) (the fused weight of bench_matmul.py:16 without fusing the
 * tensors), each member's channel tiles starting a new tile.  A plan-mode grouped call runs the
 * streaming kernel at the tiles of grid_m_max (no on-device menu).  No reference counterpart
 * (the reference fuses the weights instead).
 *   wq, ldq, sc, ld_sc, c, ldc, N  arrays of n_members entries (host memory); ldq may be NULL
 *            for wq_layout 2
 *   Other arguments as specq_w4a16, all members with the same wq_layout. */
size_t specq_w4a16_grouped_workspace_size(int m_grid, int n_members, const int* N, int K, int block_m,
                                          int block_n, int num_warps, int split_k);
/* The split count a grouped launch of these members runs (the same for every member), or 0
 * when their counts differ and they run as one launch each; the tiles a grouped call picks
 * are those specq_kernel_attrs_query reports for the members' total N with this split_k. */
int specq_w4a16_grouped_split(int n_members, const int* N, int K, int split_k);
int specq_w4a16_grouped(const void* a, int64_t lda, int n_members, const void* const* wq, const int64_t* ldq,
                        int wq_layout, const void* const* sc, const int64_t* ld_sc, void* const* c,
                        const int64_t* ldc, const int* N, int M, int K, int group, int grid_m_max,
                        const int32_t* plan, int block_m, int block_n, int num_warps, int split_k,
                        void* workspace, size_t workspace_bytes, void* stream);

/* W4A16 weight packed once at load time into 1 KB MFMA fragments (wq_layout 2 above): fragment
 * (b, t) of 128-wide K block b and 16-row tile t at (b * ceil(N/16) + t) KB; lane l's 16 bytes
 * hold row 16t + l%16 at k = 128b + 32*(l/16) + 8u + j as word u, nibble j at bits 4p..4p+3
 * with p = j/2 for even j and 4 + j/2 for odd j (rows past N hold nibble 8).  The source is layout 0 or 1 (row stride
 * ldq in elements of its storage type); `packed` holds specq_w4a16_packed_bytes() bytes, and
 * the scales stay as they are.  Results are bit-identical to layout 1 of the same weight.  No
 * reference counterpart: the reference reads the row-major packing on every call. */
size_t specq_w4a16_packed_bytes(int N, int K);
int specq_w4a16_pack_weight(const void* wq, int64_t ldq, int wq_layout, int N, int K, void* packed,
                            void* stream);

/* ---------------------------------------------------------------------------------------
 * INT8 paged-KV verification attention.
 * Replaces paged_attention (kernels.py:239-262) and _paged_attn_kernel (kernels.py:178-236).
 *   q        fp16 [B_grid, ql_grid, H, D]   strides s_qb, s_qt, s_qh (d contiguous)
 *   kc, vc   int8 [pages, PAGE, H_KV, D]    strides s_kp, s_ko, s_kh (shared by kc and vc)
 *   ks, vs   fp16 or fp32 (scale_fp32 = 0/1) [pages, PAGE, H_KV], strides s_sp, s_so, s_sh
 *   block_tbl int32 [B_grid, max_pages], row stride s_bt
 *   n_pages  pages in the K/V pool: a block-table id outside [0, n_pages) masks its page's
 *            tokens (no load; a row with no visible token left outputs 0).  No reference
 *            counterpart: the reference loads through any id it is given
 *   ctx_len  int32 [B_grid]; includes the q_len query tokens, which are the last q_len
 *            positions of each sequence (kernels.py:173, 204)
 *   out      fp16 like q, strides s_ob, s_ot, s_oh
 *   n_seqs, q_len  active sequences and query tokens (eager mode)
 *   QPP      query tokens per program: 1 = decode style, q_len = fused verification
 *            (rows packed per program = QPP * H/H_KV, at most 64)
 *   plan     NULL, or device int32*: plan[0] = n_seqs, plan[1] = q_len (the reference passes
 *            plan[1:] of its [M, B, q_len] buffer, bench_graphs.py:58)
 *   D must be 64 or 128; PAGE a multiple of 16; K/V rows 16-byte aligned with a token stride
 *   s_ko below 2^27 bytes (SPECQ_ENOTSUP otherwise).  sm_scale is the softmax scale
 *   (1/sqrt(D)).
 *   A sequence's KV range is cut into splits of whole 128-token units, their length chosen
 *   from the block table's capacity and the number of active (sequence, KV head) pairs, so a
 *   QPP=1 and a fused call, and an eager and a plan-mode call, cut a sequence at the same
 *   tokens and give bit-identical results.  In plan mode the workgroups are sized on the
 *   device to the active counts: the split count of the active sequences, and programs of
 *   only as many 16-row blocks as the active q_len fills.
 * ------------------------------------------------------------------------------------- */
size_t specq_paged_attn_workspace_size(int B_grid, int H, int H_KV, int ql_grid, int QPP,
                                       int max_pages, int PAGE);
int specq_paged_attn(const void* q, int64_t s_qb, int64_t s_qt, int64_t s_qh,
                     const int8_t* kc, const int8_t* vc, int64_t s_kp, int64_t s_ko, int64_t s_kh,
                     const void* ks, const void* vs, int64_t s_sp, int64_t s_so, int64_t s_sh,
                     int scale_fp32, const int32_t* block_tbl, int64_t s_bt, int max_pages,
                     int n_pages, const int32_t* ctx_len, void* out, int64_t s_ob, int64_t s_ot, int64_t s_oh,
                     int B_grid, int n_seqs, int q_len, int ql_grid, int H, int H_KV, int D,
                     int PAGE, int QPP, float sm_scale, const int32_t* plan,
                     void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------
 * Paged INT8 KV-cache append: quantises the q_len new tokens' K and V into the cache pages
 * that specq_paged_attn reads.  Token i of sequence b lands at position
 * pos = ctx_len[b] - q_len + i (ctx_len already counts the new tokens), page
 * block_tbl[b, pos / PAGE], slot pos % PAGE.  Each (token, KV head) row is quantised as the
 * reference builds its cache (make_paged_kv's q8, kernels.py:280-284):
 * s = max(amax |x|, 1e-8) / 127 in fp32, q = clamp(rne(x / s), -127, 127), s stored as fp16
 * (RNE) or fp32.  Replaces the host-side q8 of make_paged_kv (kernels.py:265-286) with the
 * on-device step that runs before attention in a serving loop.
 *   k_new, v_new  fp16 [B_grid, ql_grid, H_KV, D], shared strides s_nb, s_nt, s_nh
 *                 (rows 16-byte aligned).  Every workgroup of the [B_grid, ql_grid] grid
 *                 reads its new K/V row and ctx_len[b] before it checks whether b and i are
 *                 active, so k_new, v_new and ctx_len must cover all B_grid sequences and
 *                 ql_grid tokens, in eager calls (n_seqs < B_grid) as in plan mode
 *   kc, vc, ks, vs, block_tbl  as specq_paged_attn (cache rows 8-byte aligned);
 *                 n_pages = pages in the pool (rows naming a page outside [0, n_pages), or a
 *                 position outside [0, max_pages * PAGE), are skipped)
 *   plan     NULL, or device int32*: plan[0] = n_seqs, plan[1] = q_len (as specq_paged_attn)
 *   D must be 64, 128 or 256.  Slots of inactive sequences and tokens are never written.
 * ------------------------------------------------------------------------------------- */
int specq_kv_append_int8(const void* k_new, const void* v_new, int64_t s_nb, int64_t s_nt, int64_t s_nh,
                         int8_t* kc, int8_t* vc, int64_t s_kp, int64_t s_ko, int64_t s_kh,
                         void* ks, void* vs, int64_t s_sp, int64_t s_so, int64_t s_sh, int scale_fp32,
                         const int32_t* block_tbl, int64_t s_bt, int max_pages, int n_pages,
                         const int32_t* ctx_len, int B_grid, int n_seqs, int q_len, int ql_grid,
                         int H_KV, int D, int PAGE, const int32_t* plan, void* stream);

/* ---------------------------------------------------------------------------------------
 * Elementwise steps around the GEMMs of a verification layer.
 * specq_silu_mul: h[m, n] = fp16( silu(float(gate[m,n])) * float(up[m,n]) ), m < M.
 *   No reference counterpart (the reference's graph stack has no MLP activation,
 *   bench_graphs.py:62); it is the SiLU*mul step of the gate/up -> down chain.
 * specq_quantize_act_int8: per-token symmetric INT8 quantisation of fp16 rows,
 *   s[m] = max(amax_k |x[m,k]|, 1e-8) / 127,  q[m,k] = clamp(rne(x[m,k] / s[m]), -127, 127).
 *   Replaces quantize_act_int8 (kernels.py:58-62) on the device.
 * specq_silu_mul_quant_int8: the two above fused; feeds the next W8A8 GEMM directly.
 * In plan mode plan[0] is the active M.
 * ------------------------------------------------------------------------------------- */
int specq_silu_mul(const void* gate, int64_t ld_gate, const void* up, int64_t ld_up,
                   void* h, int64_t ld_h, int M, int N, int grid_m_max, const int32_t* plan,
                   void* stream);
int specq_quantize_act_int8(const void* x, int64_t ldx, int8_t* q, int64_t ldq, float* s,
                            int M, int K, int grid_m_max, const int32_t* plan, void* stream);
int specq_silu_mul_quant_int8(const void* gate, int64_t ld_gate, const void* up, int64_t ld_up,
                              int8_t* q, int64_t ldq, float* s, int M, int N, int grid_m_max,
                              const int32_t* plan, void* stream);

/* ---------------------------------------------------------------------------------------
 * Resource usage of the kernel a call with these arguments would launch (the reference's
 * compiled-kernel metadata ck.n_regs / ck.n_spills / ck.metadata.shared, regs.py:29-32).
 * kind: 0 = W8A8 (weight layout in `variant`: 0 row-major, 1 packed, 2 the packed INT4 weight
 * of W4A8), 1 = W4A16 (layout in
 * `variant`), 2 = paged attention (D in `variant`, | 1 << 16 for fp32 K/V scales).  For the GEMMs, `variant` | 16 describes a
 * call made with a plan (m_grid is then grid_m_max); a plan-mode GEMM call with automatic
 * tiles reports the tiling it runs when the active M is m_grid.
 * ------------------------------------------------------------------------------------- */
typedef struct specq_kernel_attrs {
  char name[160];          /* kernel symbol */
  int num_regs;            /* VGPRs (architected + accumulation) per lane */
  int lds_bytes;           /* LDS per workgroup (static + dynamic at these arguments) */
  int scratch_bytes;       /* private scratch per lane (register spills) */
  int threads;             /* workgroup size at these arguments */
  int grid;                /* workgroups launched at these arguments */
  int block_m, block_n, num_warps, split_k;  /* resolved tile configuration */
} specq_kernel_attrs;
int specq_kernel_attrs_query(int kind, int variant, int m_grid, int N, int K, int block_m,
                             int block_n, int num_warps, int split_k, specq_kernel_attrs* out);

#ifdef __cplusplus
}
#endif
#endif /* SPECQ_H */
