"""The reference's sweeps at the BASELINE config shapes, on the GPU, against the CPU oracle.

config 1  W8A8, every M = 1..300 x BLOCK_M in {16, 32, 64, 128} on the four Llama-3-8B
          shapes (the sweep of correctness.py:33-40 at the config shapes), row-major weights;
          load-time packed weights at the automatic tile for every M.  Bit-exact, and rows
          >= M of the output are never written.
config 2  W4A16 at every M = 1..300 (correctness.py:74's list is a subset) x BLOCK_M in {16, 32, 64, 128} on the four
          shapes, int32 packing: relative Frobenius error < 2e-3 (correctness.py:77-79) and
          the elementwise bound |out - ref| <= 2**-10 |ref| + 2e-3 rms(ref); every BLOCK_M and
          the load-time packed weight bit-identical to the automatic tile; the reference's
          uint8 packing to tolerance.
config 3  attention, B in {1, 2, 4, 8, 16, 32} x k = 0..8 at context 1024 and 4096, fp32
          scales: fused QPP = k+1 bit-identical to QPP = 1 (bench_attention.py:16-22) and
          within the bound below; plus the 49..64-row variant (QPP * G > 48) and inputs with
          large V scales.

Attention bound (stated): with A = sum_t p_t |v_t vs_t| (the oracle's magnitude),
    |out - ref| <= 2**-9 A + 2**-10 |ref| + 2**-14.
The kernel rounds each p_t * vs_t to fp16 before the PV product, as the reference does
(kernels.py:232): a relative error of at most 2**-11 per term, so at most 2**-11 A in the sum
(subnormal products add at most 2**-25 |v_t| each, covered by the 2**-14 term); the final
fp16 store adds 2**-11 |out|; fp32 accumulation and the exp2 evaluation stay far below
these.  A is measured against each term, so rows whose terms cancel are bounded correctly.
At the config-3 scales A is about 0.8, so the bound is below the reference's 2e-2
(correctness.py:100), which every case also meets.
"""
import functools

import numpy as np
import pytest
import torch

import kernels as K
from gpu_util import note
from oracle import oracle as O
from specq import gen

pytestmark = pytest.mark.gpu
DEV = "cuda"
SENT = 0x7C01            # an fp16 NaN bit pattern: no finite result has it
M_ALL = list(range(1, 301))


# ---------------------------------------------------------------------------------- config 1
@functools.lru_cache(maxsize=1)
def w8a8_case(N, Kd):
    a, w, sa, sw = gen.w8a8_inputs(300, N, Kd, seed=1000 + N + Kd)
    ref = O.w8a8(a.numpy(), sa.numpy(), w.numpy(), sw.numpy())
    dev = [t.to(DEV) for t in (a, w, sa, sw)]
    return dev, torch.from_numpy(ref.view(np.int16)).to(DEV)


def w8a8_sweep(a, sa, w, sw, ref16, bm):
    """Run every M into a sentinel-filled buffer; per-M counts of wrong and stray elements."""
    N = ref16.shape[1]
    out = torch.empty((300, N), dtype=torch.float16, device=DEV)
    outi = out.view(torch.int16)
    bad = torch.zeros(len(M_ALL), dtype=torch.int64, device=DEV)
    stray = torch.zeros(len(M_ALL), dtype=torch.int64, device=DEV)
    for i, M in enumerate(M_ALL):
        outi.fill_(SENT)
        K.w8a8_matmul(a[:M], sa[:M], w, sw, out=out[:M], BLOCK_M=bm)
        bad[i] = (outi[:M] != ref16[:M]).sum()
        stray[i] = (outi[M:] != SENT).sum()
    torch.cuda.synchronize()
    return bad.cpu().numpy(), stray.cpu().numpy()


@pytest.mark.parametrize("BM", [16, 32, 64, 128])
@pytest.mark.parametrize("shape", gen.CONFIG1_SHAPES)
def test_config1_w8a8_every_M_every_block_m(shape, BM):
    N, Kd = shape
    (a, w, sa, sw), ref16 = w8a8_case(N, Kd)
    note(f"config1 w8a8 N={N} K={Kd} BLOCK_M={BM} M=1..300")
    bad, stray = w8a8_sweep(a, sa, w, sw, ref16, BM)
    assert not bad.any(), f"fp16 mismatches at M={[M for M, b in zip(M_ALL, bad) if b][:10]}"
    assert not stray.any(), f"rows >= M written at M={[M for M, s in zip(M_ALL, stray) if s][:10]}"


@pytest.mark.parametrize("shape", gen.CONFIG1_SHAPES)
def test_config1_w8a8_packed_every_M(shape):
    N, Kd = shape
    (a, w, sa, sw), ref16 = w8a8_case(N, Kd)
    note(f"config1 w8a8 packed N={N} K={Kd} auto tile M=1..300")
    bad, stray = w8a8_sweep(a, sa, K.pack_weight_int8(w), sw, ref16, None)
    assert not bad.any(), f"fp16 mismatches at M={[M for M, b in zip(M_ALL, bad) if b][:10]}"
    assert not stray.any(), f"rows >= M written at M={[M for M, s in zip(M_ALL, stray) if s][:10]}"


# ---------------------------------------------------------------------------------- config 2
@pytest.mark.parametrize("shape", gen.CONFIG1_SHAPES)
def test_config2_w4a16_m_sweep_every_block_m(shape):
    N, Kd = shape
    qu, sc = gen.int4_weights(N, Kd, 128, seed=2000 + N + Kd)
    a = gen.fp16_acts(300, Kd, seed=3000 + N + Kd)
    ref = torch.from_numpy(O.w4a16(a.numpy(), qu.numpy(), sc.numpy(), 128)).to(DEV)
    wi = gen.pack_i32(qu).to(DEV)
    wu = gen.pack_u8_reference(qu).to(DEV)
    a, sc = a.to(DEV), sc.to(DEV)
    wpk = K.pack_weight_int4(wi)
    # Every M = 1..300 (correctness.py:74's list is a subset), as the W8A8 sweep above.
    note(f"config2 w4a16 N={N} K={Kd} {len(M_ALL)} M x BLOCK_M in (auto, 16, 32, 64, 128)")
    auto = torch.empty((300, N), dtype=torch.float16, device=DEV)
    out = torch.empty((300, N), dtype=torch.float16, device=DEV)
    fro = torch.zeros(len(M_ALL), 2, dtype=torch.float64, device=DEV)      # int32, uint8 layouts
    excess = torch.zeros(len(M_ALL), 2, dtype=torch.float64, device=DEV)
    differ = torch.zeros(len(M_ALL), dtype=torch.int64, device=DEV)

    def tol(i, j, o, r):
        e = o.double() - r
        fro[i, j] = e.norm() / r.norm()
        rms = r.square().mean().sqrt()
        excess[i, j] = (e.abs() - (2.0 ** -10 * r.abs() + 2e-3 * rms)).max()

    for i, M in enumerate(M_ALL):
        K.w4a16_matmul(a[:M], wi, sc, out=auto[:M], BLOCK_M=None)
        tol(i, 0, auto[:M], ref[:M])
        for bm in (16, 32, 64, 128):
            K.w4a16_matmul(a[:M], wi, sc, out=out[:M], BLOCK_M=bm)
            differ[i] += (out[:M] != auto[:M]).sum()
        K.w4a16_matmul(a[:M], wpk, sc, out=out[:M], BLOCK_M=None)
        differ[i] += (out[:M] != auto[:M]).sum()
        K.w4a16_matmul(a[:M], wu, sc, out=out[:M], BLOCK_M=None)
        tol(i, 1, out[:M], ref[:M])
    torch.cuda.synchronize()
    fro, excess, differ = fro.cpu().numpy(), excess.cpu().numpy(), differ.cpu().numpy()
    assert (fro < 2e-3).all(), f"rel-Frobenius {fro.max():.3e} at M={M_ALL[int(fro.max(1).argmax())]}"
    assert (excess <= 0).all(), f"elementwise bound exceeded by {excess.max():.3e}"
    assert not differ.any(), f"tiles or layouts differ from the automatic tile at M={[M for M, d in zip(M_ALL, differ) if d][:10]}"
    print(f"config2 N={N} K={Kd}: max rel-Frobenius {fro.max():.2e}")


# ---------------------------------------------------------------------------------- config 3
H, H_KV, D = 32, 8, 128


def attn_check(out, ref, mag, ql, what):
    o = out[:, :ql].float().cpu().numpy().astype(np.float64)
    r, a = ref[:, :ql], mag[:, :ql]
    err = np.abs(o - r)
    bound = 2.0 ** -9 * a + 2.0 ** -10 * np.abs(r) + 2.0 ** -14
    assert (err <= bound).all(), f"{what}: max err {err.max():.3e}, worst excess {(err - bound).max():.3e}"
    return float(err.max())


def cpu(*ts):
    return [t.cpu().numpy() for t in ts]


@pytest.mark.parametrize("B", [1, 2, 4, 8, 16, 32])
@pytest.mark.parametrize("ctx", [1024, 4096])
def test_config3_attention_grid(ctx, B):
    # One cache of ctx + 9 tokens per sequence; query length k + 1 uses ctx_len = ctx + k + 1.
    kc, vc, ks, vs, bt, cl = gen.paged_kv(B, [ctx + 9] * B, H_KV, D, seed=40 * B + ctx)
    q = gen.queries(B, 9, H, D, seed=41 * B + ctx)
    host = cpu(kc, vc, ks, vs, bt)
    kc, vc, ks, vs, bt, q = (t.to(DEV) for t in (kc, vc, ks, vs, bt, q))
    worst = 0.0
    for k in range(9):
        ql = k + 1
        cl = torch.full((B,), ctx + ql, dtype=torch.int32)
        note(f"config3 attention ctx={ctx} B={B} k={k}")
        ref, mag = O.paged_attention(q[:, :ql].cpu().numpy(), *host, cl.numpy(), ql, magnitude=True)
        cl = cl.to(DEV)
        fused, _ = K.paged_attention(q[:, :ql], kc, vc, ks, vs, bt, cl, ql, QPP=ql)
        one, _ = K.paged_attention(q[:, :ql], kc, vc, ks, vs, bt, cl, ql, QPP=1)
        torch.cuda.synchronize()
        worst = max(worst, attn_check(fused, ref, mag, ql, f"ctx={ctx} B={B} k={k}"))
        assert torch.equal(fused, one), f"QPP=1 and fused differ at ctx={ctx} B={B} k={k}"
    assert worst < 2e-2      # the reference's absolute bound (correctness.py:100)
    print(f"config3 ctx={ctx} B={B}: max abs err {worst:.2e}")


@pytest.mark.parametrize("H_q,ql", [(32, 13), (32, 16), (64, 7)])
def test_attention_rows_49_to_64(H_q, ql):
    """QPP * G in 49..64 packs four 16-row MFMA blocks (the largest program): G = 4 with 13 or 16
    query tokens, G = 8 with 7.  Tolerance, QPP=1 == fused, and plan mode == eager with
    sentinels on the inactive sequences and query slots."""
    from specq.plan import Plan
    B = 3
    ctx = [700 + ql, 1500 + ql, ql + 40]
    kc, vc, ks, vs, bt, cl = gen.paged_kv(B, ctx, H_KV, D, seed=90 + ql)
    q = gen.queries(B, ql, H_q, D, seed=91 + ql)
    ref, mag = O.paged_attention(*cpu(q, kc, vc, ks, vs, bt, cl), ql, magnitude=True)
    kc, vc, ks, vs, bt, cl, q = (t.to(DEV) for t in (kc, vc, ks, vs, bt, cl, q))
    note(f"attention {ql * H_q // H_KV} packed rows (H={H_q}, q_len={ql})")
    fused, ck = K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=ql)
    one, _ = K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=1)
    torch.cuda.synchronize()
    assert ck.config["block_m"] == 64
    attn_check(fused, ref, mag, ql, f"rows {ql * H_q // H_KV}")
    assert torch.equal(fused, one), "QPP=1 and fused differ"
    plan = Plan(DEV)
    plan.set(2, ql - 2)
    sent = torch.full_like(q, 7.0)
    K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=ql, plan=plan.attn, out=sent)
    eager = torch.full_like(q[:2], 7.0)
    K.paged_attention(q[:2], kc, vc, ks, vs, bt[:2], cl[:2], ql - 2, QPP=ql, out=eager)
    torch.cuda.synchronize()
    assert torch.equal(sent[:2], eager), "plan mode differs from eager"
    assert bool((sent[2:] == 7.0).all()) and bool((sent[:2, ql - 2:] == 7.0).all())


@pytest.mark.parametrize("k_scale", [1.0, 300.0])
def test_attention_large_v_scales(k_scale):
    """V scales in [1.5, 6] (300x config 3), so outputs reach the hundreds and rows cancel; with
    k_scale 300 the K scales grow too and the softmax becomes nearly one-hot.  The bound is
    relative to the magnitude A, so it holds whatever the cancellation."""
    B, k = 4, 8
    ql = k + 1
    kc, vc, ks, vs, bt, cl = gen.paged_kv(B, [1024 + ql, 333, 4096 + ql, 2000], H_KV, D, seed=95)
    vs = vs * 300.0
    ks = ks * k_scale
    q = gen.queries(B, ql, H, D, seed=96)
    ref, mag = O.paged_attention(*cpu(q, kc, vc, ks, vs, bt, cl), ql, magnitude=True)
    kc, vc, ks, vs, bt, cl, q = (t.to(DEV) for t in (kc, vc, ks, vs, bt, cl, q))
    note(f"attention large V scales, K scale x{k_scale}")
    fused, _ = K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=ql)
    one, _ = K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=1)
    torch.cuda.synchronize()
    attn_check(fused, ref, mag, ql, f"large V scales (K x{k_scale})")
    assert torch.equal(fused, one), "QPP=1 and fused differ"
    assert float(np.abs(ref).max()) > 50.0


def test_attention_argument_checks():
    """Bad shapes are refused on the host before any launch (nothing is read or written)."""
    kc, vc, ks, vs, bt, cl = (t.to(DEV) for t in gen.paged_kv(2, [40, 20], H_KV, D, seed=97))
    q = gen.queries(2, 3, H, D, seed=98).to(DEV)
    with pytest.raises(RuntimeError, match="n_seqs"):
        K.paged_attention(q, kc, vc, ks, vs, bt, cl, 3, n_seqs=3)
    with pytest.raises(RuntimeError, match="cover every sequence"):
        K.paged_attention(q, kc, vc, ks, vs, bt[:1], cl, 3)
    with pytest.raises(RuntimeError, match="cover every sequence"):
        K.paged_attention(q, kc, vc, ks, vs, bt, cl[:1], 3)
    with pytest.raises(RuntimeError, match="shape"):
        K.paged_attention(q, kc, vc, ks, vs, bt, cl, 3, out=torch.zeros_like(q[:1]))
    with pytest.raises(RuntimeError, match="q_len"):
        K.paged_attention(q, kc, vc, ks, vs, bt, cl, 4)
    with pytest.raises(RuntimeError, match="QPP"):
        K.paged_attention(q, kc, vc, ks, vs, bt, cl, 3, QPP=0)
