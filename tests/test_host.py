"""CPU tier: the C ABI library, its argument validation, and the host-side helpers.

No kernel is launched here: every libspecq.so call below fails validation before any HIP
call is made.
"""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "specq.h")


def header_symbols():
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\**\s+\**(specq_[a-z0-9_]+)\s*\(", txt, re.M)))


def test_header_lists_every_entry_point():
    syms = header_symbols()
    for s in ["specq_w8a8", "specq_w4a16", "specq_paged_attn", "specq_w8a8_workspace_size",
              "specq_w4a16_workspace_size", "specq_paged_attn_workspace_size", "specq_silu_mul",
              "specq_quantize_act_int8", "specq_silu_mul_quant_int8", "specq_kernel_attrs_query",
              "specq_last_error", "specq_version", "specq_kv_append_int8", "specq_w4a8_packed",
              "specq_w4a8_pack_weight", "specq_w4a8_packed_bytes", "specq_w4a8_packed_workspace_size"]:
        assert s in syms, s


def test_library_exports_every_header_symbol(built_lib):
    lib = ctypes.CDLL(built_lib)
    missing = [s for s in header_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    from specq import _lib
    assert set(_lib.SIGNATURES) >= set(header_symbols())


def test_library_loads_through_binding(built_lib):
    from specq import _lib
    assert _lib.lib().specq_version() == 100


def _w8a8_call(**kw):
    from specq import _lib
    args = dict(a=1, lda=64, w=1, ldw=64, sa=1, sw=1, c=1, ldc=32, M=4, N=32, K=64, gmm=0, plan=0,
                bm=16, bn=0, nw=4, sk=0, ws=0, wsb=0, stream=0)
    args.update(kw)
    return _lib.lib().specq_w8a8(*args.values())


def test_w8a8_validation_errors(built_lib):
    from specq import _lib
    assert _w8a8_call(a=0) == -22
    assert _w8a8_call(lda=10) == -22
    assert _w8a8_call(gmm=2) == -22            # grid_m_max < M
    assert _w8a8_call(bm=24) == -95            # BLOCK_M not a multiple of 16
    assert _w8a8_call(bm=336) == -95
    assert _w8a8_call(bn=48) == -95
    assert "BLOCK_N" in _lib.lib().specq_last_error().decode()
    # A split that needs a workspace but gets none
    assert _w8a8_call(M=16, N=32, K=8192, lda=8192, ldw=8192, sk=4) == -28


def test_w4a16_validation_errors(built_lib):
    from specq import _lib
    f = _lib.lib().specq_w4a16
    # Pointers are fake: every call below must fail validation, so nothing is launched.
    base = [16, 256, 16, 128, 0, 16, 2, 16, 64, 4, 64, 256, 128, 0, 0, 16, 0, 4, 0, 0, 0, 0]
    bad_k = list(base); bad_k[11] = 200
    assert f(*bad_k) in (-22, -95)
    bad_layout = list(base); bad_layout[4] = 3
    assert f(*bad_layout) == -22
    bad_group = list(base); bad_group[12] = 48
    assert f(*bad_group) in (-22, -95)


def test_w4a16_grouped_validation_errors(built_lib):
    import ctypes
    from specq import _lib
    L = _lib.lib()
    arr = lambda ct, vals: (ct * len(vals))(*vals)  # noqa: E731
    # Pointers are fake but aligned: every call below must fail before any launch.
    wq, ldq = arr(ctypes.c_void_p, [16 * 1024] * 3), arr(ctypes.c_int64, [512] * 3)   # int32 [N, K/8]
    sc, ldsc = arr(ctypes.c_void_p, [4096] * 3), arr(ctypes.c_int64, [32] * 3)
    c, ldc = arr(ctypes.c_void_p, [8192] * 3), arr(ctypes.c_int64, [4096, 1024, 1024])
    N = arr(ctypes.c_int, [4096, 1024, 1024])

    def call(nm=3, M=72, K=4096, group=128, layout=1):
        return L.specq_w4a16_grouped(16, K, nm, wq, ldq, layout, sc, ldsc, c, ldc, N, M, K, group, 0, None,
                                     0, 0, 4, 0, None, 0, None)
    assert call(nm=0) == -22
    assert call(nm=5) == -22
    assert "1..4" in L.specq_last_error().decode()
    assert call(layout=3) == -22               # checked per member, as the one-GEMM call does
    assert call(K=200) in (-22, -95)
    assert call(group=48) in (-22, -95)
    # q|k|v split K four ways each: the launch needs a workspace and is refused without one
    assert call() == -28
    # Workspace sizes: the split members' tiles, none for unsplit gate|up, and members whose
    # automatic split counts differ take the largest of their own calls.
    f = L.specq_w4a16_grouped_workspace_size
    assert f(72, 3, N, 4096, 0, 0, 4, 0) > 256 * 1024
    assert f(72, 0, N, 4096, 0, 0, 4, 0) == 0
    assert f(72, 2, arr(ctypes.c_int, [14336, 14336]), 4096, 0, 0, 4, 0) == 0
    assert f(72, 2, arr(ctypes.c_int, [4096, 14336]), 4096, 0, 0, 4, 0) == \
        L.specq_w4a16_workspace_size(72, 4096, 4096, 0, 0, 4, 0)


def test_attn_validation_errors(built_lib):
    from specq import _lib
    f = _lib.lib().specq_paged_attn
    args = [16, 128 * 32 * 9, 128 * 32, 128, 16, 16, 16 * 8 * 128, 8 * 128, 128, 16, 16, 128, 8, 1, 1,
            16, 64, 64, 128, 16, 16, 128 * 32 * 9, 128 * 32, 128, 2, 2, 9, 9, 32, 8, 128, 16, 9, 0.088,
            0, 0, 0, 0]
    bad_d = list(args); bad_d[30] = 96
    assert f(*bad_d) == -95
    bad_page = list(args); bad_page[31] = 8
    assert f(*bad_page) == -95
    too_many_rows = list(args); too_many_rows[32] = 17   # 17 * 4 rows > 64
    assert f(*too_many_rows) == -95
    bad_heads = list(args); bad_heads[29] = 5
    assert f(*bad_heads) == -22
    no_pool = list(args); no_pool[18] = 0
    assert f(*no_pool) == -22
    null_q = list(args); null_q[0] = 0
    assert f(*null_q) == -22


def test_kv_append_validation_errors(built_lib):
    from specq import _lib
    f = _lib.lib().specq_kv_append_int8
    # k_new, v_new, s_nb, s_nt, s_nh, kc, vc, s_kp, s_ko, s_kh, ks, vs, s_sp, s_so, s_sh, fp32,
    # bt, s_bt, max_pages, n_pages, ctx, B_grid, n_seqs, q_len, ql_grid, H_KV, D, PAGE, plan, stream
    args = [16, 16, 9 * 8 * 128, 8 * 128, 128, 16, 16, 16 * 8 * 128, 8 * 128, 128, 16, 16, 128, 8, 1, 1,
            16, 64, 64, 100, 16, 2, 2, 9, 9, 8, 128, 16, 0, 0]
    bad_d = list(args); bad_d[26] = 96
    assert f(*bad_d) == -95
    misaligned = list(args); misaligned[0] = 24
    assert f(*misaligned) == -95
    too_many = list(args); too_many[22] = 3            # n_seqs > B_grid
    assert f(*too_many) == -22
    null_bt = list(args); null_bt[16] = 0
    assert f(*null_bt) == -22
    assert f(*[a if i not in (21, 24) else 0 for i, a in enumerate(args)][:21] + [0, 0, 0, 0] + args[25:]) == 0


def test_w4a8_validation_errors(built_lib):
    from specq import _lib
    L = _lib.lib()
    assert L.specq_w4a8_packed_bytes(1000, 576) == 63 * 9 * 512
    # a, lda, w, sa, sw, c, ldc, M, N, K, gmm, plan, bm, bn, nw, sk, ws, wsb, stream
    base = [16, 131088, 16, 16, 16, 16, 32, 4, 32, 131088, 0, 0, 0, 0, 4, 0, 0, 0, 0]
    assert L.specq_w4a8_packed(*base) == -95            # K beyond the INT32 range of 16 * sum
    odd = list(base); odd[1] = odd[9] = 520
    assert L.specq_w4a8_packed(*odd) == -95             # K % 16 != 0
    assert L.specq_w4a8_pack_weight(16, 100, 2, 32, 200, 16, 0) == -22   # unknown source layout
    assert L.specq_w4a8_pack_weight(16, 10, 0, 32, 200, 16, 0) == -22    # ldq < K/2


def test_workspace_sizes(built_lib):
    from specq import _lib
    L = _lib.lib()
    assert L.specq_w8a8_workspace_size(72, 4096, 4096, 80, 32, 4, 1) == 0
    assert L.specq_w8a8_workspace_size(72, 4096, 4096, 80, 32, 4, 4) >= 256 * 1024 + 72 * 4096 * 4 * 4
    assert L.specq_w4a16_workspace_size(72, 4096, 4096, 80, 64, 4, 1) == 0
    assert L.specq_paged_attn_workspace_size(8, 32, 8, 9, 9, 8, 16) == 0   # one split
    assert L.specq_paged_attn_workspace_size(8, 32, 8, 9, 9, 257, 16) > 256 * 1024


def test_kernel_attrs_resources_file(built_lib):
    res = os.path.join(os.path.dirname(built_lib), "libspecq.resources.txt")
    txt = open(res).read()
    for name in ("w8a8_ws_kernel", "w8a8_rk_kernel", "w4a16_ws_kernel", "w4a16_rk_kernel", "paged_attn_kernel"):
        assert name in txt, name


# ---------------------------------------------------------------- host helpers vs oracle
def test_quantizers_match_oracle():
    import kernels as K
    x = torch.randn(33, 130, generator=torch.Generator().manual_seed(0)).half()
    q, s = K.quantize_act_int8(x)
    qo, so = O.quantize_rows_int8(x.numpy())
    assert np.array_equal(q.numpy(), qo) and np.array_equal(s.numpy(), so)
    q, s = K.quantize_weight_int8(x)
    assert np.array_equal(q.numpy(), qo) and np.array_equal(s.numpy(), so)


def test_int4_packer_matches_oracle():
    import kernels as K
    w = torch.randn(48, 1024, generator=torch.Generator().manual_seed(1)).half()
    p, sc, deq = K.quantize_weight_int4(w, 128)
    po, sco, deqo = O.quantize_weight_int4(w.numpy(), 128)
    assert np.array_equal(p.numpy(), po) and np.array_equal(sc.numpy(), sco)
    assert np.array_equal(deq.numpy().view(np.uint16), deqo.view(np.uint16))
    qu = O.unpack_int4_u8(po)
    assert np.array_equal(K.pack_int4_i32(torch.from_numpy(qu)).numpy(), O.pack_int4_i32(qu))


def test_generators_pack_layouts_agree():
    from specq import gen
    qu, sc = gen.int4_weights(16, 256, 128, seed=3)
    assert qu.min() >= 0 and qu.max() <= 15 and sc.dtype == torch.float16
    assert np.array_equal(O.unpack_int4_i32(gen.pack_i32(qu).numpy()), qu.numpy())
    assert np.array_equal(O.unpack_int4_u8(gen.pack_u8_reference(qu).numpy()), qu.numpy())


def test_paged_attention_ref_helper_matches_oracle():
    import kernels as K
    kc, vc, ks, vs, bt, cl = K.make_paged_kv(3, [40, 17, 33], 2, 16, device="cpu", seed=5)
    q = torch.randn(3, 4, 8, 16, generator=torch.Generator().manual_seed(6)).half()
    got = K.paged_attention_ref(q, kc, vc, ks, vs, bt, cl, 4).float().numpy()
    ref = O.paged_attention(q.numpy(), kc.numpy(), vc.numpy(), ks.numpy(), vs.numpy(), bt.numpy(), cl.numpy(), 4)
    assert np.abs(got - ref).max() < 2e-3


def test_make_paged_kv_invariants():
    import kernels as K
    kc, vc, ks, vs, bt, cl = K.make_paged_kv(4, [50, 16, 1, 33], 8, 128, device="cpu", seed=7)
    used = np.concatenate([bt[b, :(int(L) + 15) // 16].numpy() for b, L in enumerate(cl)])
    assert sorted(used.tolist()) == list(range(kc.shape[0]))      # a permutation of the pool
    assert kc.abs().max() <= 127 and ks.dtype == torch.float16
    assert (kc.abs().amax(-1) == 127).float().mean() > 0.99       # per-(page,slot,head) amax hits 127


def test_automatic_tiles_split_k_only_where_the_model_prices_it(built_lib):
    # The library's tile choice (host-side cost model, no device needed): decode tiles (M <= 16)
    # never split K, so they need no workspace; down (K = 14336) at the verification batch
    # does; and a grouped launch sizes its workspace like the fused width.
    from specq import _lib
    L = _lib.lib()
    assert L.specq_w8a8_packed_workspace_size(8, 4096, 4096, 0, 0, 4, 0) == 0
    assert L.specq_w8a8_packed_workspace_size(8, 28672, 4096, 0, 0, 4, 0) == 0
    assert L.specq_w8a8_packed_workspace_size(72, 4096, 14336, 0, 0, 4, 0) > 256 * 1024
    import ctypes
    Ns = (ctypes.c_int * 2)(14336, 14336)
    assert L.specq_w8a8_grouped_workspace_size(1, 72, 2, Ns, 4096, 0, 0, 4, 0) == \
        L.specq_w8a8_packed_workspace_size(72, 28672, 4096, 0, 0, 4, 0)
    bad = (ctypes.c_int * 2)(14336, 0)
    assert L.specq_w8a8_grouped_workspace_size(1, 72, 2, bad, 4096, 0, 0, 4, 0) == 0


def test_gpu_entry_points_refuse_cpu_tensors():
    import kernels as K
    a = torch.zeros(4, 64, dtype=torch.int8)
    with pytest.raises(RuntimeError, match="GPU"):
        K.w8a8_matmul(a, torch.ones(4), torch.zeros(8, 64, dtype=torch.int8), torch.ones(8))


def test_diag_library_is_separate(built_lib):
    """The measurement build exports its timeline and streaming-read entry points; the product
    library does not (its kernels never write timestamps)."""
    from specq import _lib
    diag = os.path.join(os.path.dirname(built_lib), "libspecq_diag.so")
    if not os.path.exists(diag):
        pytest.skip("libspecq_diag.so not built (build.py --no-diag)")
    d = ctypes.CDLL(diag)
    p = ctypes.CDLL(built_lib)
    for name in _lib.DIAG_SIGNATURES:
        assert hasattr(d, name), name
        assert not hasattr(p, name), name
    for name in header_symbols():
        assert hasattr(d, name), name


def test_bench_int4_layout_converter_matches_reference_packing():
    """bench.py's int32 -> uint8 INT4 conversion gives the reference's packing (kernels.py:143-145)."""
    import bench
    from specq import gen
    qu, _ = gen.int4_weights(40, 512, 128, seed=3)
    got = bench.i32_to_u8_reference(gen.pack_i32(qu))
    assert torch.equal(got, gen.pack_u8_reference(qu))


def test_grid_markdown_tables():
    from specq import grids
    us = {1: {0: 10.0, 8: 12.5}, 8: {0: 11.0, 8: 16.5}}
    ratio = {B: {k: us[B][k] / us[B][0] for k in us[B]} for B in us}
    md = grids.ratio_grid_md(us, ratio, "W8A8")
    assert "| 8 | 11.0 (1.00x) | 16.5 (1.50x) |" in md
    res = {(B, k, q): dict(us=float(B + k + q), frac=0.5) for B in (1, 2) for k in (0, 1) for q in ({k + 1, 1})}
    md = grids.attention_grid_md(res, 1024)
    assert "| 2 | 3.0 | 5.0 / 4.0 |" in md and "50.0 %" in md
