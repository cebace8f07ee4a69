"""Paged INT8 KV-cache append on the GPU against the CPU oracle (bit-exact).

The append quantises each (token, KV head) row exactly as the reference builds its cache
(kernels.py:280-284), so the int8 cache bytes and the stored scales (fp16 or fp32) must
match oracle.paged_kv_append bit for bit, and every slot the call does not own must keep
its previous contents.  Plan mode must equal eager and write only the active sequences and
tokens.  Appending and then attending must give the oracle's attention over the oracle's
cache.
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


def make_case(B, ctx, q_len, H_KV, D, sdtype, seed, spare_pages=3):
    """A cache filled with sentinels, a permuted block table with spare pages, and new K/V."""
    g = torch.Generator().manual_seed(seed)
    pages = [(c + 15) // 16 for c in ctx]
    total = sum(pages) + spare_pages
    perm = torch.randperm(total, generator=g).to(torch.int32)
    bt = torch.full((B, max(pages) + 1), -1, dtype=torch.int32)
    i = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[i:i + n]
        i += n
    kc = torch.randint(-127, 128, (total, 16, H_KV, D), generator=g, dtype=torch.int8)
    vc = torch.randint(-127, 128, (total, 16, H_KV, D), generator=g, dtype=torch.int8)
    ks = (torch.rand((total, 16, H_KV), generator=g) + 5).to(sdtype)
    vs = (torch.rand((total, 16, H_KV), generator=g) + 5).to(sdtype)
    k_new = (torch.randn((B, q_len, H_KV, D), generator=g) * 2).half()
    v_new = (torch.randn((B, q_len, H_KV, D), generator=g) * 2).half()
    cl = torch.tensor(ctx, dtype=torch.int32)
    return k_new, v_new, kc, vc, ks, vs, bt, cl


def to_dev(*ts):
    return [t.to(DEV) for t in ts]


def assert_cache_equal(got, ref, what):
    for name, g, r in zip(("kc", "vc", "ks", "vs"), got, ref):
        g = np.ascontiguousarray(g.cpu().numpy())
        r = np.ascontiguousarray(np.asarray(r, g.dtype))
        if not np.array_equal(g.view(np.uint8), r.view(np.uint8)):  # bytes: bit-exact scales too
            bad = np.argwhere(g != r)
            raise AssertionError(f"{what}: {name} differs at {len(bad)} places, first {tuple(bad[0])}")


@pytest.mark.parametrize("sdtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("B,ctx,q_len", [(1, [9], 9), (3, [37, 16, 300], 4), (8, [1033] * 8, 9),
                                         (5, [17, 1, 64, 65, 200], 1)])
def test_kv_append_bitexact(B, ctx, q_len, D, sdtype):
    if min(ctx) < q_len:
        pytest.skip("context shorter than the new tokens")
    H_KV = 8 if D <= 128 else 2
    case = make_case(B, ctx, q_len, H_KV, D, sdtype, seed=B * 1000 + D + q_len)
    k_new, v_new, kc, vc, ks, vs, bt, cl = case
    ref = O.paged_kv_append(k_new.numpy(), v_new.numpy(), kc.numpy(), vc.numpy(), ks.numpy(), vs.numpy(),
                            bt.numpy(), cl.numpy(), q_len)
    note(f"kv_append B={B} ctx={ctx[:3]} q_len={q_len} D={D} {sdtype}")
    k_new, v_new, kc, vc, ks, vs, bt, cl = to_dev(*case)
    K.paged_kv_append(k_new, v_new, kc, vc, ks, vs, bt, cl, q_len)
    torch.cuda.synchronize()
    assert_cache_equal((kc, vc, ks, vs), ref, f"B={B} q_len={q_len} D={D}")


def test_kv_append_strided_new_kv():
    # K and V as views into one fused [B, q_len, 2, H_KV, D] projection output.
    B, ctx, q_len, H_KV, D = 4, [40, 33, 70, 19], 5, 8, 128
    k_new, v_new, kc, vc, ks, vs, bt, cl = make_case(B, ctx, q_len, H_KV, D, torch.float32, seed=77)
    fused = torch.stack([k_new, v_new], dim=2)
    ref = O.paged_kv_append(k_new.numpy(), v_new.numpy(), kc.numpy(), vc.numpy(), ks.numpy(), vs.numpy(),
                            bt.numpy(), cl.numpy(), q_len)
    note("kv_append strided views")
    fused, kc, vc, ks, vs, bt, cl = to_dev(fused, kc, vc, ks, vs, bt, cl)
    K.paged_kv_append(fused[:, :, 0], fused[:, :, 1], kc, vc, ks, vs, bt, cl, q_len)
    torch.cuda.synchronize()
    assert_cache_equal((kc, vc, ks, vs), ref, "strided")


def test_kv_append_plan_mode_matches_eager_and_leaves_inactive_slots():
    B, QL, H_KV, D = 6, 9, 8, 128
    ctx_full = [300, 41, 129, 16, 77, 500]
    for n_seqs, q_len in [(6, 9), (3, 4), (1, 1), (0, 3), (4, 0)]:
        # ctx_len counts the new tokens: each sequence's context ends q_len past its base.
        ctx = [c - (QL - q_len) for c in ctx_full]
        case = make_case(B, ctx_full, QL, H_KV, D, torch.float16, seed=11 + n_seqs)
        k_new, v_new, kc, vc, ks, vs, bt, _ = case
        cl = torch.tensor(ctx, dtype=torch.int32)
        ref = O.paged_kv_append(k_new.numpy(), v_new.numpy(), kc.numpy(), vc.numpy(), ks.numpy(), vs.numpy(),
                                bt.numpy(), cl.numpy(), q_len, n_seqs=n_seqs)
        note(f"kv_append plan n_seqs={n_seqs} q_len={q_len}")
        k_new, v_new, kc, vc, ks, vs, bt, cl = to_dev(k_new, v_new, kc, vc, ks, vs, bt, cl)
        plan = torch.tensor([n_seqs, q_len], dtype=torch.int32, device=DEV)
        K.paged_kv_append(k_new, v_new, kc, vc, ks, vs, bt, cl, plan=plan)
        torch.cuda.synchronize()
        assert_cache_equal((kc, vc, ks, vs), ref, f"plan n_seqs={n_seqs} q_len={q_len}")


def test_kv_append_then_attention_matches_oracle():
    # The serving order: write the k+1 new tokens, then verify them against the whole cache.
    B, k, H, H_KV, D = 4, 8, 32, 8, 128
    ql = k + 1
    ctx = [1024 + ql, 300 + ql, 16 + ql, 777 + ql]
    # the config-3 cache (scales U[0.005, 0.02]) holds the context; the new rows are N(0, 1)
    kc, vc, ks, vs, bt, cl = gen.paged_kv(B, ctx, H_KV, D, seed=5)
    g = torch.Generator().manual_seed(6)
    k_new = torch.randn((B, ql, H_KV, D), generator=g).half()
    v_new = torch.randn((B, ql, H_KV, D), generator=g).half()
    q = gen.queries(B, ql, H, D, seed=7)
    rk, rv, rks, rvs = O.paged_kv_append(k_new.numpy(), v_new.numpy(), kc.numpy(), vc.numpy(), ks.numpy(),
                                         vs.numpy(), bt.numpy(), cl.numpy(), ql)
    ref = O.paged_attention(q.numpy(), rk, rv, rks, rvs, bt.numpy(), cl.numpy(), ql)
    note("kv_append then attention")
    k_new, v_new, kc, vc, ks, vs, bt, cl, q = to_dev(k_new, v_new, kc, vc, ks, vs, bt, cl, q)
    K.paged_kv_append(k_new, v_new, kc, vc, ks, vs, bt, cl, ql)
    out, _ = K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy().astype(np.float64)
    err = np.abs(o - ref)
    assert (err <= 4e-3 + 2.0 ** -9 * np.abs(ref)).all(), f"max err {err.max():.3e}"


def test_kv_append_rejects_bad_arguments():
    k_new, v_new, kc, vc, ks, vs, bt, cl = to_dev(*make_case(2, [20, 20], 2, 8, 96 + 32, torch.float16, seed=1))
    with pytest.raises(RuntimeError):
        K.paged_kv_append(k_new[..., :96], v_new[..., :96], kc[..., :96], vc[..., :96], ks, vs, bt, cl, 2)
    with pytest.raises(RuntimeError):
        K.paged_kv_append(k_new, v_new, kc.view(torch.uint8), vc, ks, vs, bt, cl, 2)
