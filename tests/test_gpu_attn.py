"""INT8 paged verification attention on the GPU against the float64 CPU oracle.

Tolerance (stated): max |out - ref| <= 4e-3 + 2**-9 * |ref| elementwise, well inside the
reference's 2e-2 (correctness.py:100).  The kernel's deviations from the exact float64
result are the fp16 rounding of p * vs before the PV product (as the reference,
kernels.py:232), fp32 accumulation, exp2 rounding and the final fp16 store.
Bit-exact properties: QPP=1 and fused QPP=k+1 give identical outputs; plan mode equals
eager and leaves inactive sequences / query slots untouched.
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
H, H_KV, D = 32, 8, 128


def check(out, ref, ql, what):
    o = out[:, :ql].float().cpu().numpy().astype(np.float64)
    r = ref[:, :ql]
    err = np.abs(o - r)
    bound = 4e-3 + 2.0 ** -9 * np.abs(r)
    assert (err <= bound).all(), f"{what}: max err {err.max():.3e}"
    return float(err.max())


def cpu(*ts):
    return [t.cpu().numpy() for t in ts]


@pytest.mark.parametrize("B", [1, 3, 8])
@pytest.mark.parametrize("k", [2, 4, 8])
def test_attention_correctness_py_cases(B, k):
    # correctness.py:89-100: random context in [k+1, 700), reference generator, QPP in {1, k+1}
    ql = k + 1
    g = torch.Generator().manual_seed(100 * B + k)
    ctx = [int(x) for x in torch.randint(ql, 700, (B,), generator=g)]
    kc, vc, ks, vs, bt, cl = K.make_paged_kv(B, ctx, H_KV, D, device=DEV, seed=B * 10 + k)
    q = torch.randn(B, ql, H, D, generator=g).half().to(DEV)
    ref = O.paged_attention(*cpu(q, kc, vc, ks, vs, bt, cl), ql)
    note(f"attn B={B} k={k} ctx={ctx}")
    outs = {}
    for QPP in (1, ql):
        out, _ = K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=QPP)
        torch.cuda.synchronize()
        check(out, ref, ql, f"B={B} k={k} QPP={QPP}")
        outs[QPP] = out
    assert torch.equal(outs[1], outs[ql]), "QPP=1 and fused results differ"


@pytest.mark.parametrize("ctx", [1024, 4096])
@pytest.mark.parametrize("k", [0, 3, 8])
def test_attention_config3_fp32_scales(ctx, k):
    B, ql = 8, k + 1
    note(f"attn config3 B={B} ctx={ctx} k={k}")
    kc, vc, ks, vs, bt, cl = gen.paged_kv(B, [ctx + ql] * B, H_KV, D, seed=ctx + k)
    q = gen.queries(B, ql, H, D, seed=k)
    ref = O.paged_attention(*cpu(q, kc, vc, ks, vs, bt, cl), ql)
    kc, vc, ks, vs, bt, cl, q = (t.to(DEV) for t in (kc, vc, ks, vs, bt, cl, q))
    o1, _ = K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=ql)
    o2, _ = K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=1)
    torch.cuda.synchronize()
    check(o1, ref, ql, "fused")
    assert torch.equal(o1, o2)


def test_attention_plan_mode_sentinels():
    # correctness.py:103-120: one grid (B_MAX=8, QLMAX=9), active (B, q_len) from plan[1:3].
    BMAX, QLMAX = 8, 9
    g = torch.Generator().manual_seed(99)
    ctx = [int(x) for x in torch.randint(QLMAX, 700, (BMAX,), generator=g)]
    kc, vc, ks, vs, bt, cl = K.make_paged_kv(BMAX, ctx, H_KV, D, device=DEV, seed=99)
    qfull = torch.randn(BMAX, QLMAX, H, D, generator=g).half().to(DEV)
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    for B_act, ql in ((1, 3), (3, 5), (8, 9), (5, 3), (8, 5), (0, 4), (8, 1)):
        note(f"attn plan B={B_act} ql={ql}")
        plan[1], plan[2] = B_act, ql
        out = torch.full_like(qfull, 7.0)
        K.paged_attention(qfull, kc, vc, ks, vs, bt, cl, QLMAX, QPP=QLMAX, plan=plan[1:], out=out)
        torch.cuda.synchronize()
        if B_act:
            eager = torch.full_like(qfull[:B_act], 7.0)
            K.paged_attention(qfull[:B_act], kc, vc, ks, vs, bt[:B_act], cl[:B_act], ql, QPP=ql, out=eager)
            torch.cuda.synchronize()
            assert torch.equal(out[:B_act, :ql], eager[:, :ql])
            ref = O.paged_attention(*cpu(qfull[:B_act], kc, vc, ks, vs, bt[:B_act], cl[:B_act]), ql)
            check(out[:B_act], ref, ql, f"plan B={B_act} ql={ql}")
        assert bool((out[B_act:] == 7.0).all()) and bool((out[:B_act, ql:] == 7.0).all())


def test_attention_head_dim_64_and_no_visible_key():
    note("attn D=64, L < q_len")
    kc, vc, ks, vs, bt, cl = gen.paged_kv(2, [600, 2], 4, 64, seed=3, scale_dtype=torch.float16)
    q = gen.queries(2, 4, 16, 64, seed=4)
    cl[1] = 2  # only 2 tokens but 4 queries: the first two query rows see no key -> 0
    ref = O.paged_attention(*cpu(q, kc, vc, ks, vs, bt, cl), 4)
    kc, vc, ks, vs, bt, cl, q = (t.to(DEV) for t in (kc, vc, ks, vs, bt, cl, q))
    out, _ = K.paged_attention(q, kc, vc, ks, vs, bt, cl, 4)
    torch.cuda.synchronize()
    check(out, ref, 4, "D=64")
    assert bool((out[1, :2] == 0).all())


def test_attention_long_context_sub_splits():
    """A block table beyond 64 x 512 tokens makes each workgroup cover several 512-token
    sub-splits; results stay within tolerance and QPP=1 still equals the fused program."""
    B, k = 2, 3
    ql = k + 1
    ctx = [33000 + ql, 20000 + ql]   # the block table spans ~33K tokens for both sequences
    kc, vc, ks, vs, bt, cl = gen.paged_kv(B, ctx, H_KV, D, seed=71)
    q = gen.queries(B, ql, H, D, seed=72)
    ref = O.paged_attention(*cpu(q, kc, vc, ks, vs, bt, cl), ql)
    kc, vc, ks, vs, bt, cl, q = (t.to(DEV) for t in (kc, vc, ks, vs, bt, cl, q))
    note(f"attn long context ctx={ctx} max_pages={bt.shape[1]}")
    outs = {}
    for QPP in (1, ql):
        out, _ = K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=QPP)
        torch.cuda.synchronize()
        check(out, ref, ql, f"long ctx QPP={QPP}")
        outs[QPP] = out
    assert torch.equal(outs[1], outs[ql]), "QPP=1 and fused results differ"


def test_attention_page32_ragged_and_plan_subset():
    """PAGE=32 (two 16-token sub-tiles per page), ragged contexts from the query tokens alone to
    1290 tokens, fp16 scales; QPP=1 equals fused, and a plan-mode call with 3 of 5 sequences
    active equals eager on those 3 and leaves the others untouched."""
    B, k = 5, 3
    ql = k + 1
    ctx = [ql, 9, 33, 517, 1290]
    kc, vc, ks, vs, bt, cl = gen.paged_kv(B, ctx, H_KV, D, PAGE=32, seed=81, scale_dtype=torch.float16)
    q = gen.queries(B, ql, H, D, seed=82)
    ref = O.paged_attention(*cpu(q, kc, vc, ks, vs, bt, cl), ql)
    kc, vc, ks, vs, bt, cl, q = (t.to(DEV) for t in (kc, vc, ks, vs, bt, cl, q))
    note(f"attn PAGE=32 ragged ctx={ctx}")
    outs = {}
    for QPP in (1, ql):
        out, _ = K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=QPP)
        torch.cuda.synchronize()
        check(out, ref, ql, f"PAGE=32 QPP={QPP}")
        outs[QPP] = out
    assert torch.equal(outs[1], outs[ql]), "QPP=1 and fused results differ"
    from specq.plan import Plan
    plan = Plan(DEV)
    plan.set(3, ql)
    sentinel = torch.full_like(q, 7.0)
    K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=ql, plan=plan.attn, out=sentinel)
    torch.cuda.synchronize()
    eager3, _ = K.paged_attention(q[:3], kc, vc, ks, vs, bt[:3], cl[:3], ql, QPP=ql)
    torch.cuda.synchronize()
    assert torch.equal(sentinel[:3], eager3), "plan mode differs from eager on the active sequences"
    assert bool((sentinel[3:] == 7.0).all()), "plan mode wrote inactive sequences"


def test_attention_single_sequence_many_splits():
    """One sequence of 9000 tokens: the split length targets the CU count, so the sequence is
    cut into more than 16 splits (the merge's second weight pass); QPP=1 equals fused."""
    B, k = 1, 8
    ql = k + 1
    kc, vc, ks, vs, bt, cl = gen.paged_kv(B, [9000 + ql], H_KV, D, seed=83)
    q = gen.queries(B, ql, H, D, seed=84)
    ref = O.paged_attention(*cpu(q, kc, vc, ks, vs, bt, cl), ql)
    kc, vc, ks, vs, bt, cl, q = (t.to(DEV) for t in (kc, vc, ks, vs, bt, cl, q))
    note("attn B=1 ctx=9000 many splits")
    o1, _ = K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=ql)
    o2, _ = K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=1)
    torch.cuda.synchronize()
    check(o1, ref, ql, "B=1 ctx=9000")
    assert torch.equal(o1, o2)


@pytest.mark.parametrize("target", [32, 4096])
def test_attention_split_target_option(target):
    """The attn_target_wgs option moves the split length (32: the longest splits, 4096: the
    shortest).  Results stay within tolerance; QPP=1 equals fused and a plan-mode call equals
    eager at the same setting."""
    from specq import _lib
    from specq.plan import Plan
    B, k = 3, 4
    ql = k + 1
    ctx = [700, 2100, 3333]
    kc, vc, ks, vs, bt, cl = gen.paged_kv(B, ctx, H_KV, D, seed=85)
    q = gen.queries(B, ql, H, D, seed=86)
    ref = O.paged_attention(*cpu(q, kc, vc, ks, vs, bt, cl), ql)
    kc, vc, ks, vs, bt, cl, q = (t.to(DEV) for t in (kc, vc, ks, vs, bt, cl, q))
    note(f"attn split target {target}")
    _lib.set_option("attn_target_wgs", target)
    try:
        o1, _ = K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=ql)
        o2, _ = K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=1)
        plan = Plan(DEV)
        plan.set(B, ql)
        o3 = torch.full_like(q, 7.0)
        K.paged_attention(q, kc, vc, ks, vs, bt, cl, ql, QPP=ql, plan=plan.attn, out=o3)
        torch.cuda.synchronize()
    finally:
        _lib.set_option("attn_target_wgs", 0)
    check(o1, ref, ql, f"target {target}")
    assert torch.equal(o1, o2), "QPP=1 and fused results differ"
    assert torch.equal(o1, o3), "plan mode differs from eager"


@pytest.mark.parametrize("D_, PAGE, sdt", [(128, 16, torch.float32), (64, 32, torch.float16)])
def test_attention_out_of_pool_page_ids(D_, PAGE, sdt):
    """Block-table ids outside [0, pages) mask their page's tokens (n_pages bound, no load):
    sequence 0 has three scattered bad prefix pages (ids = pages, -1, 2^31 - 1), sequence 1 a
    run of bad pages over 1440 tokens that empties whole splits, sequence 2 only bad pages.  Expected:
    the oracle on the block table with the bad pages removed (context shortened by as many
    pages; the query tokens' pages stay valid, so causal positions keep their order), and
    zeros for sequence 2.  QPP=1 equals fused, and plan mode equals eager."""
    from specq.plan import Plan
    B, k = 3, 4
    ql = k + 1
    ctx = [1500, 3000, 200]
    kc, vc, ks, vs, bt, cl = gen.paged_kv(B, ctx, H_KV, D_, PAGE=PAGE, seed=87, scale_dtype=sdt)
    q = gen.queries(B, ql, H, D_, seed=88)
    n_pages = kc.shape[0]
    run = 90 * 16 // PAGE  # 1440 tokens of bad pages in sequence 1
    bad = {0: {2: n_pages, 5: -1, 6: 2**31 - 1}, 1: {j: n_pages + j for j in range(10, 10 + run)}}
    bt_bad = bt.clone()
    bt_ok = torch.zeros_like(bt)
    cl_ok = cl.clone()
    for b in range(B):
        used = (ctx[b] + PAGE - 1) // PAGE
        if b == 2:
            bt_bad[b, :used] = n_pages + 1000
            continue
        keep = [int(bt[b, j]) for j in range(used) if j not in bad[b]]
        for j, v in bad[b].items():
            assert (j + 1) * PAGE <= ctx[b] - ql, "bad pages must be whole prefix pages"
            bt_bad[b, j] = v
        bt_ok[b, :len(keep)] = torch.tensor(keep, dtype=torch.int32)
        cl_ok[b] = ctx[b] - PAGE * len(bad[b])
    ref = O.paged_attention(*cpu(q, kc, vc, ks, vs, bt_ok, cl_ok), ql)
    ref[2] = 0.0
    kc, vc, ks, vs, bt_bad, cl, q = (t.to(DEV) for t in (kc, vc, ks, vs, bt_bad, cl, q))
    note(f"attn out-of-pool page ids D={D_} PAGE={PAGE} ctx={ctx} n_pages={n_pages}")
    outs = {}
    for QPP in (1, ql):
        out, _ = K.paged_attention(q, kc, vc, ks, vs, bt_bad, cl, ql, QPP=QPP)
        torch.cuda.synchronize()
        check(out, ref, ql, f"out-of-pool ids QPP={QPP}")
        outs[QPP] = out
    assert torch.equal(outs[1], outs[ql]), "QPP=1 and fused results differ"
    assert bool((outs[ql][2] == 0).all()), "a sequence with only out-of-pool pages must give zeros"
    plan = Plan(DEV)
    plan.set(B, ql)
    o3 = torch.full_like(q, 7.0)
    K.paged_attention(q, kc, vc, ks, vs, bt_bad, cl, ql, QPP=ql, plan=plan.attn, out=o3)
    torch.cuda.synchronize()
    assert torch.equal(o3, outs[ql]), "plan mode differs from eager"
