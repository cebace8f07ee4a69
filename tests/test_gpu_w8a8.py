"""W8A8 GEMM on the GPU against the CPU oracle: bit-exact fp16 outputs (INT32 accumulation
and the fp32 epilogue in the reference order are exact), every M = 1..300 at every
BLOCK_M, the config-1 Llama shapes, plan mode with sentinel rows, split-K invariance."""
import numpy as np
import pytest
import torch

import kernels as K
from gpu_util import assert_bitexact_fp16, note
from oracle import oracle as O
from specq import gen

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def odd_case():
    # correctness.py:28-31: N=1000, K=520, deliberately not tile multiples.
    torch.manual_seed(0)
    w = torch.randn(1000, 520, dtype=torch.float16)
    w_q, sw = K.quantize_weight_int8(w)
    x_all = torch.randn(300, 520, dtype=torch.float16)
    a_q, sa = K.quantize_act_int8(x_all)  # per-token: rows do not depend on M
    ref = O.w8a8(a_q.numpy(), sa.numpy(), w_q.numpy(), sw.numpy())
    return [t.to(DEV) for t in (a_q, sa, w_q, sw)], ref


@pytest.mark.parametrize("BM", [16, 32, 64, 128])
def test_w8a8_every_M_every_block_m_odd_shape(odd_case, BM):
    (a_q, sa, w_q, sw), ref = odd_case
    note(f"w8a8 N=1000 K=520 BLOCK_M={BM} M=1..300")
    outs = [K.w8a8_matmul(a_q[:M], sa[:M], w_q, sw, BLOCK_M=BM)[0] for M in range(1, 301)]
    torch.cuda.synchronize()
    for M, out in zip(range(1, 301), outs):
        assert_bitexact_fp16(out, ref[:M], f"BLOCK_M={BM} M={M}")


def test_w8a8_every_M_auto_tile_aligned():
    note("w8a8 N=1000 K=512 auto BLOCK_M M=1..300")
    a, w, sa, sw = gen.w8a8_inputs(300, 1000, 512, seed=11)
    ref = O.w8a8(a.numpy(), sa.numpy(), w.numpy(), sw.numpy())
    a, w, sa, sw = (t.to(DEV) for t in (a, w, sa, sw))
    outs = [K.w8a8_matmul(a[:M], sa[:M], w, sw, BLOCK_M=None)[0] for M in range(1, 301)]
    torch.cuda.synchronize()
    for M, out in zip(range(1, 301), outs):
        assert_bitexact_fp16(out, ref[:M], f"auto M={M}")


@pytest.mark.parametrize("shape", gen.CONFIG1_SHAPES)
def test_w8a8_config1_shapes(shape):
    N, Kd = shape
    Ms = [1, 8, 20, 72, 160, 288, 300]
    note(f"w8a8 config1 N={N} K={Kd} M={Ms}")
    a, w, sa, sw = gen.w8a8_inputs(300, N, Kd, seed=1000 + N + Kd)
    ref = O.w8a8(a.numpy(), sa.numpy(), w.numpy(), sw.numpy())
    a, w, sa, sw = (t.to(DEV) for t in (a, w, sa, sw))
    for M in Ms:
        for bm in (None, 16, 128):
            out, ck = K.w8a8_matmul(a[:M], sa[:M], w, sw, BLOCK_M=bm)
            torch.cuda.synchronize()
            assert_bitexact_fp16(out, ref[:M], f"N={N} K={Kd} M={M} BLOCK_M={bm}")
    assert ck.n_spills == 0


def test_w8a8_config0_and_int32_kat():
    note("w8a8 config0 M=20 K=N=4096 + all-127 KAT")
    a, w, sa, sw = gen.w8a8_inputs(20, 4096, 4096, seed=0)
    ref = O.w8a8(a.numpy(), sa.numpy(), w.numpy(), sw.numpy())
    out, _ = K.w8a8_matmul(a.to(DEV), sa.to(DEV), w.to(DEV), sw.to(DEV), BLOCK_M=None)
    assert_bitexact_fp16(out, ref, "config0")
    # acc = 16129 * 4096 > 2**24: an fp32 accumulator would round it.
    a127 = torch.full((5, 4096), 127, dtype=torch.int8, device=DEV)
    w127 = torch.full((64, 4096), 127, dtype=torch.int8, device=DEV)
    sa1 = torch.full((5,), 2.0 ** -20, device=DEV)
    sw1 = torch.ones(64, device=DEV)
    out, _ = K.w8a8_matmul(a127, sa1, w127, sw1, BLOCK_M=None)
    want = np.float16(np.float32(16129 * 4096) * np.float32(2.0 ** -20))
    assert (out.cpu().numpy() == want).all()


@pytest.mark.parametrize("split_k", [1, 2, 3, 7, 16])
def test_w8a8_split_k_and_tiles_bit_identical(split_k):
    note(f"w8a8 split_k={split_k}")
    a, w, sa, sw = gen.w8a8_inputs(72, 4096, 4096, seed=5)
    ref = O.w8a8(a.numpy(), sa.numpy(), w.numpy(), sw.numpy())
    a, w, sa, sw = (t.to(DEV) for t in (a, w, sa, sw))
    for bn, nw in ((16, 4), (32, 2), (64, 1), (32, 4), (64, 2), (128, 4)):
        out, _ = K.w8a8_matmul(a, sa, w, sw, BLOCK_M=80, BLOCK_N=bn, num_warps=nw, split_k=split_k)
        torch.cuda.synchronize()
        assert_bitexact_fp16(out, ref, f"split_k={split_k} BLOCK_N={bn} warps={nw}")


def test_w8a8_epilogue_fp32_rounding_order():
    # Every channel has an output whose fp32 product sits on an fp16 rounding midpoint, so an
    # epilogue that rounds the product to fp16 once (fused multiply-convert) fails here.  N is
    # ragged, so the 4-channel vector stores and the per-channel edge stores are both covered.
    N = 1003
    note(f"w8a8 epilogue rounding order M=96 N={N} K=64")
    a, w, sa, sw, hit = gen.w8a8_epilogue_midpoints(96, N, seed=7)
    assert bool(hit.any(dim=0).all())
    ref = O.w8a8(a.numpy(), sa.numpy(), w.numpy(), sw.numpy())
    a, w, sa, sw = (t.to(DEV) for t in (a, w, sa, sw))
    wp = K.pack_weight_int8(w)
    for M in (16, 96):
        for wt, bm, bn, nw, sk in ((w, None, None, 4, 0), (w, 16, 16, 4, 0), (w, 80, 64, 4, 0), (w, 96, 32, 4, 3),
                                   (wp, None, None, 4, 0), (wp, 96, 128, 4, 0), (wp, 16, 16, 4, 2)):
            out, ck = K.w8a8_matmul(a[:M], sa[:M], wt, sw, BLOCK_M=bm, BLOCK_N=bn, num_warps=nw, split_k=sk)
            torch.cuda.synchronize()
            assert_bitexact_fp16(out, ref[:M], f"M={M} BLOCK_M={bm} BLOCK_N={bn} sk={sk} ({ck.name})")


@pytest.mark.parametrize("bn_nw", [(16, 4), (32, 4), (32, 2), (64, 4), (64, 2), (128, 4)])
def test_w8a8_every_tile_shape_and_block_m(bn_nw):
    # Every channel-block shape of the aligned streaming paths at every BLOCK_M bucket,
    # including the deep tiles that change the K-chunk length.
    bn, nw = bn_nw
    note(f"w8a8 tile sweep BLOCK_N={bn} warps={nw}")
    a, w, sa, sw = gen.w8a8_inputs(300, 1000, 1536, seed=31)
    ref = O.w8a8(a.numpy(), sa.numpy(), w.numpy(), sw.numpy())
    a, w, sa, sw = (t.to(DEV) for t in (a, w, sa, sw))
    for bm in (16, 32, 48, 80, 144, 192, 208, 288, 304):
        for M in sorted({1, min(bm, 300), min(bm + 5, 300), 300}):
            out, ck = K.w8a8_matmul(a[:M], sa[:M], w, sw, BLOCK_M=bm, BLOCK_N=bn, num_warps=nw)
            torch.cuda.synchronize()
            assert_bitexact_fp16(out, ref[:M], f"BLOCK_N={bn} warps={nw} BLOCK_M={bm} M={M} ({ck.name})")


@pytest.mark.parametrize("shape", [(1000, 1536)] + gen.CONFIG1_SHAPES)
def test_w8a8_packed_weight_bit_exact(shape):
    N, Kd = shape
    note(f"w8a8 packed weight N={N} K={Kd}")
    a, w, sa, sw = gen.w8a8_inputs(300, N, Kd, seed=41 + N)
    ref = O.w8a8(a.numpy(), sa.numpy(), w.numpy(), sw.numpy())
    a, w, sa, sw = (t.to(DEV) for t in (a, w, sa, sw))
    wp = K.pack_weight_int8(w)
    for M in (1, 8, 72, 300):
        for bn, nw, sk in ((None, 4, 0), (16, 4, 0), (32, 2, 3), (16, 1, 0)):
            out, _ = K.w8a8_matmul(a[:M], sa[:M], wp, sw, BLOCK_M=None, BLOCK_N=bn, num_warps=nw, split_k=sk)
            torch.cuda.synchronize()
            assert_bitexact_fp16(out, ref[:M], f"packed N={N} K={Kd} M={M} bn={bn} nw={nw} sk={sk}")


@pytest.mark.parametrize("path", [1, 2, 3])
def test_w8a8_kernel_families_bit_identical(path):
    # w8a8_path 1: direct-activation streaming kernel (16-row token tiles), 2: LDS-staged
    # activations (deeper tiles), 3: byte-granular legacy kernel.  All sum the same INT32s.
    from specq import _lib
    note(f"w8a8 kernel family {path}")
    a, w, sa, sw = gen.w8a8_inputs(300, 1000, 1536, seed=51)
    ref = O.w8a8(a.numpy(), sa.numpy(), w.numpy(), sw.numpy())
    a, w, sa, sw = (t.to(DEV) for t in (a, w, sa, sw))
    _lib.set_option("w8a8_path", path)
    try:
        for M in (1, 17, 72, 300):
            for bm in (None, 16, 64):
                for bn in (None, 16, 32, 64, 128):
                    out, ck = K.w8a8_matmul(a[:M], sa[:M], w, sw, BLOCK_M=bm, BLOCK_N=bn, num_warps=4)
                    torch.cuda.synchronize()
                    assert_bitexact_fp16(out, ref[:M], f"path={path} M={M} BLOCK_M={bm} BLOCK_N={bn} ({ck.name})")
    finally:
        _lib.set_option("w8a8_path", 0)


@pytest.mark.parametrize("layout", [0, 1])
def test_w8a8_streaming_tiles_and_layouts(layout):
    # Streaming kernels (direct and LDS-staged activations): tile depths from 16 to 304 rows,
    # every channel width, K tails that are not whole 256-byte chunks, N tails, explicit
    # split-K, row-major and packed weights.
    for N, Kd in ((1000, 1552), (4096, 4096)):
        note(f"w8a8 streaming layout={layout} N={N} K={Kd}")
        a, w, sa, sw = gen.w8a8_inputs(300, N, Kd, seed=61 + N)
        ref = O.w8a8(a.numpy(), sa.numpy(), w.numpy(), sw.numpy())
        a, w, sa, sw = (t.to(DEV) for t in (a, w, sa, sw))
        wt = K.pack_weight_int8(w) if layout == 1 else w
        for bm in (None, 16, 32, 80, 160, 256, 304):
            for M in (1, 17, 72, 130, 300):
                for bn, sk in ((None, 0), (16, 0), (32, 2), (64, 1), (128, 0), (64, 3), (16, 5)):
                    out, ck = K.w8a8_matmul(a[:M], sa[:M], wt, sw, BLOCK_M=bm, BLOCK_N=bn, split_k=sk)
                    torch.cuda.synchronize()
                    assert_bitexact_fp16(out, ref[:M], f"streaming N={N} K={Kd} M={M} BLOCK_M={bm} "
                                                       f"BLOCK_N={bn} sk={sk} ({ck.name})")


def test_w8a8_plan_mode_sentinel_rows():
    # correctness.py:50-65: fixed grid at M_MAX=288, active M from plan[0], rows >= M untouched.
    note("w8a8 plan mode M_MAX=288")
    torch.manual_seed(1)
    a, w, sa, sw = gen.w8a8_inputs(288, 1000, 520, seed=21)
    ref = O.w8a8(a.numpy(), sa.numpy(), w.numpy(), sw.numpy())
    a, w, sa, sw = (t.to(DEV) for t in (a, w, sa, sw))
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    for bm in (16, 128, 288):
        for M in (1, 3, 5, 9, 15, 16, 17, 27, 45, 81, 144, 288, 0):
            plan[0] = M
            out = torch.full((288, 1000), 12345.0, device=DEV, dtype=torch.float16)
            K.w8a8_matmul(a, sa, w, sw, out=out, plan=plan, grid_m_max=288, BLOCK_M=bm)
            torch.cuda.synchronize()
            assert_bitexact_fp16(out[:M], ref[:M], f"plan BLOCK_M={bm} M={M}")
            assert bool((out[M:] == 12345.0).all()), f"rows >= M={M} were written (BLOCK_M={bm})"
    # plan values beyond the grid are clamped to it
    plan[0] = 10_000
    out = torch.full((288, 1000), 12345.0, device=DEV, dtype=torch.float16)
    K.w8a8_matmul(a, sa, w, sw, out=out, plan=plan, grid_m_max=288, BLOCK_M=64)
    torch.cuda.synchronize()
    assert_bitexact_fp16(out, ref, "plan clamp")


def test_w8a8_deterministic_and_strided_out():
    note("w8a8 determinism + strided output")
    a, w, sa, sw = (t.to(DEV) for t in gen.w8a8_inputs(40, 1024, 4096, seed=9))
    o1, _ = K.w8a8_matmul(a, sa, w, sw, BLOCK_M=None)
    o2, _ = K.w8a8_matmul(a, sa, w, sw, BLOCK_M=None)
    big = torch.full((40, 1500), 7.0, dtype=torch.float16, device=DEV)
    K.w8a8_matmul(a, sa, w, sw, out=big[:, 200:1224], BLOCK_M=None)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(big[:, 200:1224], o1)
    assert bool((big[:, :200] == 7.0).all()) and bool((big[:, 1224:] == 7.0).all())

