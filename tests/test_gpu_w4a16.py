"""W4A16 GEMM on the GPU against the float64 CPU oracle.

Tolerance (stated): the kernel rounds fp16 weights exactly like the reference and sums
exact fp16 x fp16 products in fp32, so its error is the final fp16 rounding plus fp32
accumulation: elementwise |out - ref| <= 2**-10 * |ref| + 2e-3 * rms(ref), and the
reference's own criterion, relative Frobenius error < 2e-3 (correctness.py:77-79).
Plan mode is bit-identical to eager and never writes rows >= M.
"""
import numpy as np
import pytest
import torch

import kernels as K
from gpu_util import note
from oracle import oracle as O
from specq import gen

pytestmark = pytest.mark.gpu
DEV = "cuda"


def check_tol(out, ref, what):
    o = out.float().cpu().numpy().astype(np.float64)
    rms = float(np.sqrt(np.mean(ref ** 2))) or 1.0
    err = np.abs(o - ref)
    bound = 2.0 ** -10 * np.abs(ref) + 2e-3 * rms
    fro = float(np.linalg.norm(o - ref) / (np.linalg.norm(ref) or 1.0))
    assert (err <= bound).all(), f"{what}: max excess {float((err - bound).max())} (rms {rms})"
    assert fro < 2e-3, f"{what}: rel-Frobenius {fro}"
    return fro


@pytest.fixture(scope="module")
def ref_case():
    # correctness.py:68-71: N=1000, K=1024, group 128, weights from the reference quantizer.
    torch.manual_seed(0)
    w4 = torch.randn(1000, 1024, dtype=torch.float16)
    wp, sc, deq = K.quantize_weight_int4(w4, group=128)
    x4 = torch.randn(300, 1024, dtype=torch.float16)
    qu = O.unpack_int4_u8(wp.numpy())
    ref = O.w4a16(x4.numpy(), qu, sc.numpy(), 128)
    return x4.to(DEV), wp.to(DEV), sc.to(DEV), qu, ref


MS = list(range(1, 65)) + [72, 99, 128, 129, 200, 288, 300]


@pytest.mark.parametrize("BM", [16, 32, 64, 128])
def test_w4a16_reference_layout_m_sweep(ref_case, BM):
    x4, wp, sc, _, ref = ref_case
    note(f"w4a16 layout0 N=1000 K=1024 BLOCK_M={BM}")
    outs = [K.w4a16_matmul(x4[:M], wp, sc, BLOCK_M=BM)[0] for M in MS]
    torch.cuda.synchronize()
    worst = 0.0
    for M, out in zip(MS, outs):
        worst = max(worst, check_tol(out, ref[:M], f"BLOCK_M={BM} M={M}"))
    print(f"max rel-Frobenius {worst:.2e}")


def test_w4a16_int32_layout_and_auto_tile(ref_case):
    x4, _, sc, qu, ref = ref_case
    note("w4a16 layout1 auto BLOCK_M")
    wi = torch.from_numpy(O.pack_int4_i32(qu)).to(DEV)
    outs = [K.w4a16_matmul(x4[:M], wi, sc, BLOCK_M=None)[0] for M in MS]
    torch.cuda.synchronize()
    for M, out in zip(MS, outs):
        check_tol(out, ref[:M], f"layout1 M={M}")


@pytest.mark.parametrize("shape", gen.CONFIG1_SHAPES)
def test_w4a16_config2_shapes(shape):
    N, Kd = shape
    note(f"w4a16 config2 N={N} K={Kd}")
    qu, sc = gen.int4_weights(N, Kd, 128, seed=2000 + N)
    a = gen.fp16_acts(300, Kd, seed=3000 + Kd)
    ref = O.w4a16(a.numpy(), qu.numpy(), sc.numpy(), 128)
    wi = gen.pack_i32(qu).to(DEV)
    wu = gen.pack_u8_reference(qu).to(DEV)
    a, sc = a.to(DEV), sc.to(DEV)
    for M in (1, 8, 72, 300):
        for wp in (wi, wu):
            out, ck = K.w4a16_matmul(a[:M], wp, sc, BLOCK_M=None)
            torch.cuda.synchronize()
            check_tol(out, ref[:M], f"N={N} K={Kd} M={M} {wp.dtype}")
    assert ck.n_spills == 0


def test_w4a16_kats():
    note("w4a16 KATs")
    a = gen.fp16_acts(16, 256, seed=1).to(DEV)
    zero_u8 = torch.full((64, 128), 0x88, dtype=torch.uint8, device=DEV)
    sc = torch.full((64, 2), 0.01, dtype=torch.float16, device=DEV)
    out, _ = K.w4a16_matmul(a, zero_u8, sc, BLOCK_M=None)
    assert bool((out == 0).all())
    one = zero_u8.clone()
    one[5, 17] = 0x8D            # k = 17 holds q = +5 (low nibble); k = 145 stays 0
    out, _ = K.w4a16_matmul(a, one, sc, BLOCK_M=None)
    w = np.float16(np.float16(5.0) * np.float16(0.01))
    want = (a[:, 17].float().cpu().numpy() * np.float32(w)).astype(np.float16)
    assert np.array_equal(out[:, 5].cpu().numpy(), want)
    assert bool((out[:, :5] == 0).all()) and bool((out[:, 6:] == 0).all())


def test_w4a16_plan_mode_bit_identical_to_eager():
    note("w4a16 plan mode")
    qu, sc = gen.int4_weights(4096, 4096, 128, seed=7)
    wi, sc = gen.pack_i32(qu).to(DEV), sc.to(DEV)
    a = gen.fp16_acts(288, 4096, seed=8).to(DEV)
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    for bm in (16, 128):
        for M in (1, 9, 27, 72, 288):
            eager, _ = K.w4a16_matmul(a[:M], wi, sc, BLOCK_M=bm)
            plan[0] = M
            out = torch.full((288, 4096), 7.0, dtype=torch.float16, device=DEV)
            K.w4a16_matmul(a, wi, sc, out=out, plan=plan, grid_m_max=288, BLOCK_M=bm)
            torch.cuda.synchronize()
            assert torch.equal(out[:M], eager), f"plan != eager at BLOCK_M={bm} M={M}"
            assert bool((out[M:] == 7.0).all())
    # the fp32 summation order does not depend on BLOCK_M either
    e16, _ = K.w4a16_matmul(a[:100], wi, sc, BLOCK_M=16)
    e128, _ = K.w4a16_matmul(a[:100], wi, sc, BLOCK_M=128)
    torch.cuda.synchronize()
    assert torch.equal(e16, e128)


def _pack(wp):
    out = K.pack_weight_int4(wp)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("shape", [(1000, 1024), (4096, 4096), (1024, 4096), (4096, 14336), (17, 256), (1, 128),
                                   (33, 384), (70, 640)])
def test_w4a16_layouts_families_tiles_bit_identical(shape):
    """Every kernel family (w4a16_path 1: register stream, 2: LDS-staged), BLOCK_M and
    BLOCK_N gives the same bits, and so do the layouts that walk K in the same order (int32
    and packed, whichever layout it was packed from); the reference uint8 layout pairs k with
    k + K/2 in each byte, so its blocks cover other k and it has its own order.  Every result
    meets the tolerance against the oracle."""
    from specq import _lib
    N, Kd = shape
    note(f"w4a16 layouts/families/tiles N={N} K={Kd}")
    qu, sc = gen.int4_weights(N, Kd, 128, seed=40 + N)
    a = gen.fp16_acts(300, Kd, seed=41 + Kd)
    ref = O.w4a16(a.numpy(), qu.numpy(), sc.numpy(), 128)
    wu, wi = gen.pack_u8_reference(qu).to(DEV), gen.pack_i32(qu).to(DEV)
    a, sc = a.to(DEV), sc.to(DEV)
    weights = {"u8": ("u8", wu), "i32": ("k", wi), "packed(u8)": ("k", _pack(wu)), "packed(i32)": ("k", _pack(wi))}
    try:
        for M in (1, 5, 16, 17, 32, 72, 100, 300):
            base = {}
            for path in (0, 1, 2):
                _lib.set_option("w4a16_path", path)
                for wname, (order, wp) in weights.items():
                    for bm in (None, 16, 32, 80, 160, 256):
                        for bn in (None, 128):
                            out, ck = K.w4a16_matmul(a[:M], wp, sc, BLOCK_M=bm, BLOCK_N=bn)
                            torch.cuda.synchronize()
                            what = f"M={M} path={path} {wname} BLOCK_M={bm} BLOCK_N={bn} ({ck.name})"
                            if order not in base:
                                base[order] = out
                                check_tol(out, ref[:M], what)
                            else:
                                assert torch.equal(out, base[order]), what
    finally:
        _lib.set_option("w4a16_path", 0)


@pytest.mark.parametrize("group", [16, 32, 64, 256])
def test_w4a16_group_sizes(group):
    """Group sizes other than 128 (scales change within a 128-wide K block for groups below 128,
    and every two blocks for 256): every layout that supports the group (16 only with the
    reference uint8 layout), both kernel families and a plan-mode call, against the oracle;
    the layouts that walk K in the same order give the same bits."""
    from specq import _lib
    N, Kd = 200, 1024
    note(f"w4a16 group={group}")
    qu, sc = gen.int4_weights(N, Kd, group, seed=60 + group)
    a = gen.fp16_acts(100, Kd, seed=61)
    ref = O.w4a16(a.numpy(), qu.numpy(), sc.numpy(), group)
    a, sc = a.to(DEV), sc.to(DEV)
    weights = {"u8": ("u8", gen.pack_u8_reference(qu).to(DEV))}
    if group >= 32:
        wi = gen.pack_i32(qu).to(DEV)
        weights.update({"i32": ("k", wi), "packed": ("k", _pack(wi))})
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    try:
        for M in (1, 17, 72, 100):
            base = {}
            for path in (1, 2):
                _lib.set_option("w4a16_path", path)
                for wname, (order, wp) in weights.items():
                    for bm in (None, 16, 32, 80):
                        out, ck = K.w4a16_matmul(a[:M], wp, sc, group=group, BLOCK_M=bm, BLOCK_K=min(64, group))
                        torch.cuda.synchronize()
                        what = f"group={group} M={M} path={path} {wname} BLOCK_M={bm} ({ck.name})"
                        if order not in base:
                            base[order] = out
                            check_tol(out, ref[:M], what)
                        else:
                            assert torch.equal(out, base[order]), what
            _lib.set_option("w4a16_path", 0)
            for wname, (order, wp) in weights.items():
                plan[0] = M
                outp = torch.full((100, N), 7.0, dtype=torch.float16, device=DEV)
                K.w4a16_matmul(a, wp, sc, group=group, out=outp, plan=plan, grid_m_max=100, BLOCK_M=None,
                               BLOCK_K=min(64, group))
                torch.cuda.synchronize()
                assert torch.equal(outp[:M], base[order]), f"group={group} {wname}: plan mode differs at M={M}"
                assert bool((outp[M:] == 7.0).all()), f"group={group} {wname}: plan mode wrote rows >= M"
    finally:
        _lib.set_option("w4a16_path", 0)


@pytest.mark.parametrize("split_k", [1, 2, 3])
def test_w4a16_odd_block_counts_per_split(split_k):
    """K = 640 is 5 blocks: splits of 5, 3 + 2 and 2 + 2 + 1 blocks, so the odd-index stream of
    a split is one block short or empty.  Both kernel families, every BLOCK_M, the same bits;
    within tolerance of the oracle."""
    from specq import _lib
    N, Kd = 200, 640
    note(f"w4a16 odd blocks split_k={split_k}")
    qu, sc = gen.int4_weights(N, Kd, 128, seed=57)
    a = gen.fp16_acts(100, Kd, seed=58)
    ref = O.w4a16(a.numpy(), qu.numpy(), sc.numpy(), 128)
    wi, a, sc = gen.pack_i32(qu).to(DEV), a.to(DEV), sc.to(DEV)
    try:
        for M in (1, 16, 17, 100):
            base = None
            for path in (1, 2):
                _lib.set_option("w4a16_path", path)
                for bm in (16, 32, 48, 144):
                    out, ck = K.w4a16_matmul(a[:M], wi, sc, BLOCK_M=bm, split_k=split_k)
                    torch.cuda.synchronize()
                    what = f"M={M} path={path} BLOCK_M={bm} split_k={split_k} ({ck.name})"
                    if base is None:
                        base = out
                        check_tol(out, ref[:M], what)
                    else:
                        assert torch.equal(out, base), what
    finally:
        _lib.set_option("w4a16_path", 0)


@pytest.mark.parametrize("split_k", [1, 2, 3, 5, 8])
def test_w4a16_explicit_split_k(split_k):
    N, Kd = 1024, 4096
    note(f"w4a16 split_k={split_k}")
    qu, sc = gen.int4_weights(N, Kd, 128, seed=55)
    a = gen.fp16_acts(80, Kd, seed=56)
    ref = O.w4a16(a.numpy(), qu.numpy(), sc.numpy(), 128)
    wi, a, sc = gen.pack_i32(qu).to(DEV), a.to(DEV), sc.to(DEV)
    for M in (1, 8, 80):
        outs = [K.w4a16_matmul(a[:M], wi, sc, BLOCK_M=bm, split_k=split_k)[0] for bm in (16, 80)]
        torch.cuda.synchronize()
        check_tol(outs[0], ref[:M], f"split_k={split_k} M={M}")
        assert torch.equal(outs[0], outs[1])


def test_w4a16_packed_plan_mode_graph_replays():
    """Plan-mode W4A16 on the packed layout inside a captured graph: every replay matches the
    eager call bit for bit and rows >= M stay untouched."""
    note("w4a16 packed plan graph")
    N, Kd, MMAX = 4096, 4096, 288
    qu, sc = gen.int4_weights(N, Kd, 128, seed=61)
    wpk = _pack(gen.pack_i32(qu).to(DEV))
    sc = sc.to(DEV)
    a = gen.fp16_acts(MMAX, Kd, seed=62).to(DEV)
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    out = torch.full((MMAX, N), 7.0, dtype=torch.float16, device=DEV)
    plan[0] = MMAX
    K.w4a16_matmul(a, wpk, sc, out=out, plan=plan, grid_m_max=MMAX, BLOCK_M=None)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g):
            K.w4a16_matmul(a, wpk, sc, out=out, plan=plan, grid_m_max=MMAX, BLOCK_M=None)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for M in (72, 1, 288, 9, 150, 72):
        out.fill_(7.0)
        plan[0] = M
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        eager, _ = K.w4a16_matmul(a[:M], wpk, sc, BLOCK_M=None)
        torch.cuda.synchronize()
        assert torch.equal(out[:M], eager), f"replay M={M}"
        assert bool((out[M:] == 7.0).all()), f"replay M={M} wrote rows >= M"
