"""W4A8 GEMM on the GPU: INT4 weights on the INT8 MFMA path, per-channel scale in the epilogue.

The INT32 sums are exact, so the fp16 outputs must be bit-identical to the CPU oracle (W8A8 on
the unpacked weight) at small sizes and to the GPU W8A8 kernel on the unpacked int8 weight at
the config-1 Llama sizes (W8A8 is itself pinned bit-exact against the oracle).  Covered: every
tile family and channel width, K and N tails, split-K, both source packings, plan mode with
sentinel rows, and the INT32 range limit of the 16x-scaled sums (K = 131072).
"""
import numpy as np
import pytest
import torch

import kernels as K
from gpu_util import assert_bitexact_fp16, note
from oracle import oracle as O
from specq import gen

pytestmark = pytest.mark.gpu
DEV = "cuda"


def w4a8_case(M, N, Kd, seed):
    a, sa = gen.w8a8_acts(M, Kd, seed=seed)
    qu, _ = gen.int4_weights(N, Kd, group=Kd, seed=seed + 1)
    sw = (torch.rand(N, generator=torch.Generator().manual_seed(seed + 2)) * 0.009 + 0.001).float()
    return a, sa, qu, sw


@pytest.mark.parametrize("N,Kd", [(1000, 576), (1003, 1552), (4096, 4096)])
def test_w4a8_bitexact_vs_oracle(N, Kd):
    a, sa, qu, sw = w4a8_case(300, N, Kd, seed=N + Kd)
    ref = O.w4a8(a.numpy(), sa.numpy(), qu.numpy(), sw.numpy())
    note(f"w4a8 N={N} K={Kd}")
    a, sa, sw = a.to(DEV), sa.to(DEV), sw.to(DEV)
    wp = K.pack_weight_w4a8(gen.pack_u8_reference(qu).to(DEV))
    for M in (1, 2, 15, 16, 17, 33, 72, 100, 144, 200, 288, 300):
        for bm, bn, sk in ((None, None, 0), (16, None, 0), (32, 16, 2), (80, 64, 0), (128, 128, 3),
                           (304, 32, 0), (None, 16, 5)):
            out, ck = K.w4a8_matmul(a[:M], sa[:M], wp, sw, BLOCK_M=bm, BLOCK_N=bn, split_k=sk)
            torch.cuda.synchronize()
            assert_bitexact_fp16(out, ref[:M], f"w4a8 N={N} K={Kd} M={M} BLOCK_M={bm} BLOCK_N={bn} "
                                               f"sk={sk} ({ck.name})")


@pytest.mark.parametrize("shape", gen.CONFIG1_SHAPES)
def test_w4a8_config1_shapes_equal_w8a8_on_unpacked_weight(shape):
    N, Kd = shape
    a, sa, qu, sw = w4a8_case(300, N, Kd, seed=7 * N + Kd)
    note(f"w4a8 config1 N={N} K={Kd}")
    a, sa, sw, qu = a.to(DEV), sa.to(DEV), sw.to(DEV), qu.to(DEV)
    w8 = (qu.to(torch.int16) - 8).to(torch.int8)
    wp = K.pack_weight_w4a8(gen.pack_i32(qu))
    wp8 = K.pack_weight_int8(w8)
    for M in (1, 8, 20, 72, 160, 288, 300):
        ref, _ = K.w8a8_matmul(a[:M], sa[:M], wp8, sw, BLOCK_M=None)
        out, ck = K.w4a8_matmul(a[:M], sa[:M], wp, sw, BLOCK_M=None)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"M={M} ({ck.name})"
    # one point against the CPU oracle at full size
    M = 72
    ref = O.w4a8(a[:M].cpu().numpy(), sa[:M].cpu().numpy(), qu.cpu().numpy(), sw.cpu().numpy())
    out, _ = K.w4a8_matmul(a[:M], sa[:M], wp, sw, BLOCK_M=None)
    torch.cuda.synchronize()
    assert_bitexact_fp16(out, ref, f"w4a8 config1 N={N} K={Kd} M=72 vs oracle")


def test_w4a8_source_layouts_and_unpacked_call_agree():
    N, Kd = 520, 1024
    a, sa, qu, sw = w4a8_case(40, N, Kd, seed=3)
    note("w4a8 u8 / int32 sources")
    a, sa, sw, qu = a.to(DEV), sa.to(DEV), sw.to(DEV), qu.to(DEV)
    o1, _ = K.w4a8_matmul(a, sa, K.pack_weight_w4a8(gen.pack_u8_reference(qu)), sw)
    o2, _ = K.w4a8_matmul(a, sa, K.pack_weight_w4a8(gen.pack_i32(qu)), sw)
    o3, _ = K.w4a8_matmul(a, sa, gen.pack_u8_reference(qu), sw)  # packed inside the call
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(o1, o3)


def test_w4a8_int32_range_limit_kat():
    # a = -127, q = -8 everywhere: sum = 1016 * K; at K = 131072 the kernel's 16x-scaled sum is
    # 2,130,706,432, just inside INT32.  One more 16-wide step is rejected.
    Kd = 131072
    note("w4a8 K=131072 KAT")
    a = torch.full((3, Kd), -127, dtype=torch.int8, device=DEV)
    qu = torch.zeros((32, Kd), dtype=torch.uint8, device=DEV)
    qu[1::2] = 15  # +7 on odd channels: sum = -889 * K
    sa = torch.ones(3, device=DEV)
    sw = torch.full((32,), 2.0 ** -24, device=DEV)
    out, _ = K.w4a8_matmul(a, sa, gen.pack_u8_reference(qu), sw, BLOCK_M=None)
    torch.cuda.synchronize()
    # closed form: 1016 * K * 2**-24 = 7.9375 and -889 * K * 2**-24 = -6.9453125, exact in fp16
    want = torch.tensor([1016.0 if n % 2 == 0 else -889.0 for n in range(32)]) * Kd / 2.0 ** 24
    assert torch.equal(out.float().cpu(), want.expand(3, 32)), out[0, :4]
    a2 = torch.zeros((1, Kd + 16), dtype=torch.int8, device=DEV)
    with pytest.raises(RuntimeError):
        K.w4a8_matmul(a2, sa[:1], torch.zeros((32, (Kd + 16) // 2), dtype=torch.uint8, device=DEV), sw)


def test_w4a8_plan_mode_sentinel_rows():
    N, Kd = 1000, 576
    a, sa, qu, sw = w4a8_case(288, N, Kd, seed=31)
    ref = O.w4a8(a.numpy(), sa.numpy(), qu.numpy(), sw.numpy())
    note("w4a8 plan mode M_MAX=288")
    a, sa, sw = a.to(DEV), sa.to(DEV), sw.to(DEV)
    wp = K.pack_weight_w4a8(gen.pack_u8_reference(qu).to(DEV))
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    for bm in (16, 128, None):
        for M in (1, 9, 16, 17, 72, 144, 288, 0):
            plan[0] = M
            out = torch.full((288, N), 12345.0, device=DEV, dtype=torch.float16)
            K.w4a8_matmul(a, sa, wp, sw, out=out, plan=plan, grid_m_max=288, BLOCK_M=bm)
            torch.cuda.synchronize()
            assert_bitexact_fp16(out[:M], ref[:M], f"w4a8 plan BLOCK_M={bm} M={M}")
            assert bool((out[M:] == 12345.0).all()), f"rows >= M={M} were written (BLOCK_M={bm})"
