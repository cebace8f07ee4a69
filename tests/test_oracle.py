"""Pins for the CPU oracle (oracle/oracle.py), each independent of the oracle's formula.

The reference ships no golden vectors (its results/correctness.json holds scalar maxima
only), so every oracle function is pinned by what the mathematics fixes:
  w8a8_int32         torch._int_mm (library), pure-Python brute force, all-127 closed form
  w8a8               torch fp32 epilogue in the reference order; closed-form KAT; a
                     reordered epilogue is shown to differ (the order is really tested)
  quantize_rows_int8 hand-computed KATs incl. round-half-to-even and the 1e-8 clamp;
                     torch restatement (library round)
  int4 pack/unpack   byte KATs 0x88 -> (0, 0), 0x0F -> (+7, -8); exhaustive round trips;
                     u8 <-> int32 layouts agree on every nibble
  quantize_weight_int4  hand-worked packed bytes, fp16 scales and fp32-scale dequantised
                     values (incl. half to even, the 1e-8 clamp, the j / j + K/2 pairing)
  dequant / w4a16    all-0x88 -> 0; single nonzero nibble -> a[:, k] * (q - 8) * s; torch
                     float64 matmul
  paged_attention    torch scaled_dot_product_attention in float64 (library) on a dense
                     gather; brute-force Python softmax; constant-V and single-key closed
                     forms; invariance under a consistent pool permutation
  silu_mul           torch.nn.functional.silu
  cpu_baseline.*     the torch formulas bench.py times on the host: bit-exact (W8A8) or to
                     tolerance (W4A16, attention) against the pinned numpy oracle above
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- W8A8
def test_w8a8_int32_matches_torch_int_mm():
    r = rng(0)
    a = r.integers(-127, 128, (32, 520), dtype=np.int8)
    w = r.integers(-127, 128, (1000, 520), dtype=np.int8)
    ref = torch._int_mm(torch.from_numpy(a), torch.from_numpy(w).T.contiguous()).numpy()
    assert np.array_equal(O.w8a8_int32(a, w), ref)


def test_w8a8_int32_brute_force_tiny():
    r = rng(1)
    a = r.integers(-127, 128, (3, 7), dtype=np.int8)
    w = r.integers(-127, 128, (5, 7), dtype=np.int8)
    got = O.w8a8_int32(a, w)
    for m in range(3):
        for n in range(5):
            assert got[m, n] == sum(int(a[m, k]) * int(w[n, k]) for k in range(7))


def test_w8a8_all_127_closed_form_exceeds_fp32_exact_range():
    K = 4096
    a = np.full((2, K), 127, np.int8)
    w = np.full((3, K), -127, np.int8)
    acc = O.w8a8_int32(a, w)
    assert (acc == -16129 * K).all() and 16129 * K > 2 ** 24


def test_w8a8_epilogue_matches_torch_reference_order():
    r = rng(2)
    a = r.integers(-127, 128, (20, 256), dtype=np.int8)
    w = r.integers(-127, 128, (64, 256), dtype=np.int8)
    sa = r.uniform(0.005, 0.02, 20).astype(np.float32)
    sw = r.uniform(0.001, 0.01, 64).astype(np.float32)
    acc = torch._int_mm(torch.from_numpy(a), torch.from_numpy(w).T.contiguous())
    ref = ((acc.float() * torch.from_numpy(sa)[:, None]) * torch.from_numpy(sw)[None, :]).half().numpy()
    got = O.w8a8(a, sa, w, sw)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    # The order matters: acc * (sa * sw) rounds differently somewhere in this block.
    other = (acc.float() * (torch.from_numpy(sa)[:, None] * torch.from_numpy(sw)[None, :])).half().numpy()
    assert not np.array_equal(other.view(np.uint16), ref.view(np.uint16))


def test_w8a8_epilogue_rounds_through_fp32():
    # Cases where the fp32 product lands on an fp16 rounding midpoint: the reference order
    # rounds to fp32 and then to fp16; a single rounding of the exact product (what a fused
    # multiply-convert does) differs on every marked element.
    from specq import gen
    a, w, sa, sw, hit = (t.numpy() for t in gen.w8a8_epilogue_midpoints(16, 160, seed=3))
    assert hit.any(axis=0).all()
    acc = O.w8a8_int32(a, w)
    ref = ((torch.from_numpy(acc).float() * torch.from_numpy(sa)[:, None]) * torch.from_numpy(sw)[None, :]).half().numpy()
    got = O.w8a8(a, sa, w, sw)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    once = ((acc.astype(np.float32) * sa[:, None]).astype(np.float64) * sw[None, :].astype(np.float64)).astype(np.float16)
    assert (got.view(np.uint16) != once.view(np.uint16))[hit].all()


def test_w8a8_kat_single_term():
    a = np.zeros((1, 64), np.int8); a[0, 5] = 100
    w = np.zeros((2, 64), np.int8); w[1, 5] = -3
    out = O.w8a8(a, np.array([0.5], np.float32), w, np.array([1.0, 0.25], np.float32))
    assert out[0, 0] == 0 and out[0, 1] == np.float16(-300 * 0.5 * 0.25)


# ---------------------------------------------------------------- quantisers
def test_quantize_rows_kats():
    x = np.array([[127.0, -63.5, 0.5, 1.5, 2.5, -2.5, 0.0]], np.float32)
    q, s = O.quantize_rows_int8(x)
    assert s[0] == np.float32(1.0)
    assert q.tolist() == [[127, -64, 0, 2, 2, -2, 0]]  # half-to-even at .5
    z, sz = O.quantize_rows_int8(np.zeros((1, 4), np.float32))
    assert sz[0] == np.float32(1e-8) / np.float32(127.0) and (z == 0).all()


def test_quantize_rows_matches_torch_formula():
    x = torch.randn(40, 300, generator=torch.Generator().manual_seed(3)).half()
    s_t = x.abs().amax(-1).float().clamp(min=1e-8) / 127.0
    q_t = torch.round(x.float() / s_t[:, None]).clamp(-127, 127).to(torch.int8)
    q, s = O.quantize_rows_int8(x.numpy())
    assert np.array_equal(q, q_t.numpy()) and np.array_equal(s, s_t.numpy())


# ---------------------------------------------------------------- INT4
def test_int4_byte_kats():
    assert O.unpack_int4_u8(np.array([[0x88]], np.uint8)).astype(int).tolist() == [[8, 8]]
    lo_hi = O.unpack_int4_u8(np.array([[0x0F]], np.uint8)).astype(int) - 8
    assert lo_hi.tolist() == [[7, -8]]


def test_int4_round_trips_exhaustive():
    vals = np.array(np.meshgrid(np.arange(16), np.arange(16))).reshape(2, -1).T  # all nibble pairs
    qu = np.concatenate([vals[:, :1], vals[:, 1:]], axis=1).astype(np.uint8).reshape(1, -1)
    qu = np.concatenate([qu, qu[:, ::-1]], axis=0)  # [2, 512]
    assert np.array_equal(O.unpack_int4_u8(O.pack_int4_u8(qu)), qu)
    assert np.array_equal(O.unpack_int4_i32(O.pack_int4_i32(qu)), qu)
    words = O.pack_int4_i32(np.arange(8, dtype=np.uint8).reshape(1, 8))
    assert words.view(np.uint32)[0, 0] == 0x76543210


def test_int4_quantizer_known_answers():
    # Hand-worked case of kernels.py:138-147 with group 4 (K = 16, K/2 = 8 holds two groups).
    #   row 0, group 0: amax 7 -> sc = 1 exactly; 7, 3.5, -2.5, 0.5 -> 7, 4, -2, 0 (half to even)
    #   row 0, group 1: all zero -> sc = 1e-8 / 7 (fp16: 0), q = 0
    #   row 0, group 2: amax 0.7 -> sc = fp32(0.1); -0.7, 0.12, 0.33, -0.04 -> -7, 1, 3, 0
    #   row 0, group 3: amax 0.014 -> sc = fp32(0.002); 0, -0.0031, 0.0062, 0.014 -> 0, -2, 3, 7
    #   row 1: amax 7 in every group, integer weights -> q = w
    w = np.array([[7.0, 3.5, -2.5, 0.5, 0, 0, 0, 0, -0.7, 0.12, 0.33, -0.04, 0.0, -0.0031, 0.0062, 0.014],
                  [-7, -6, -5, -4, 7, 6, 5, 4, 1, 2, 3, 7, -1, -2, -3, 7]], np.float32)
    packed, sc, deq = O.quantize_weight_int4(w, 4)
    # byte j holds k = j in its low nibble and k = j + 8 in its high nibble, each as q + 8
    assert packed.tolist() == [[0x1F, 0x9C, 0xB6, 0x88, 0x88, 0x68, 0xB8, 0xF8],
                               [0x91, 0xA2, 0xB3, 0xF4, 0x7F, 0x6E, 0x5D, 0xFC]]
    # fp16 scales: 1, 1e-8/7 underflows to 0, fp16(0.1), fp16(0.002)
    assert sc.astype(np.float64).tolist() == [[1.0, 0.0, 0.0999755859375, 0.0020008087158203125], [1.0] * 4]
    # deq = fp16(q * sc) with the fp32 scale: -7 * fp32(0.1) -> -0.7001953125, where the fp16
    # scale would give -0.69970703125 (and 3 -> 0.300048828125 against 0.2998046875)
    assert deq[0].astype(np.float64).tolist() == [7.0, 4.0, -2.0, 0.0, 0.0, 0.0, 0.0, 0.0,
                                                  -0.7001953125, 0.0999755859375, 0.300048828125, 0.0,
                                                  0.0, -0.004001617431640625, 0.006000518798828125,
                                                  0.01399993896484375]
    assert deq[1].astype(np.float64).tolist() == w[1].astype(np.float64).tolist()
    # |w / sc| <= 7 always, so nibbles stay in 1..15 (the -8 clamp is never reached)
    big = np.random.default_rng(3).standard_normal((16, 256)).astype(np.float32)
    nib = O.unpack_int4_u8(O.quantize_weight_int4(big, 128)[0])
    assert nib.min() >= 1 and nib.max() <= 15
    with pytest.raises(AssertionError):
        O.quantize_weight_int4(np.zeros((1, 24), np.float32), 8)     # (K/2) % group != 0


def test_w4a16_kats_and_torch():
    r = rng(5)
    N, K, G = 32, 256, 128
    a = r.standard_normal((4, K)).astype(np.float16)
    zero = O.w4a16(a, np.full((N, K), 8, np.uint8), np.ones((N, K // G), np.float16), G)
    assert (zero == 0).all()
    qu = np.full((N, K), 8, np.uint8); qu[3, 200] = 8 + 5
    sc = np.full((N, K // G), 0.0123, np.float16)
    one = O.w4a16(a, qu, sc, G)
    expect = a[:, 200].astype(np.float64) * float(np.float16(5 * np.float32(np.float16(0.0123))))
    assert np.array_equal(one[:, 3], expect) and (np.delete(one, 3, axis=1) == 0).all()
    qu = r.integers(0, 16, (N, K)).astype(np.uint8)
    sc = r.uniform(0.002, 0.02, (N, K // G)).astype(np.float16)
    deq_t = ((torch.from_numpy(qu.astype(np.int16)) - 8).half() * torch.from_numpy(sc).repeat_interleave(G, 1)).double()
    ref = torch.from_numpy(a).double() @ deq_t.T
    assert np.allclose(O.w4a16(a, qu, sc, G), ref.numpy(), rtol=0, atol=1e-12)


# ---------------------------------------------------------------- attention
def _small_cache(seed, B=2, ctx=(37, 20), H=8, H_KV=2, D=16, PAGE=16):
    r = rng(seed)
    pages = [(c + PAGE - 1) // PAGE for c in ctx]
    total = sum(pages)
    perm = r.permutation(total)
    bt = np.zeros((B, max(pages)), np.int32)
    i = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[i:i + n]; i += n
    kc = r.integers(-127, 128, (total, PAGE, H_KV, D), dtype=np.int8)
    vc = r.integers(-127, 128, (total, PAGE, H_KV, D), dtype=np.int8)
    ks = r.uniform(0.005, 0.02, (total, PAGE, H_KV)).astype(np.float32)
    vs = r.uniform(0.005, 0.02, (total, PAGE, H_KV)).astype(np.float32)
    return kc, vc, ks, vs, bt, np.array(ctx, np.int32)


def test_attention_matches_torch_sdpa_float64():
    kc, vc, ks, vs, bt, cl = _small_cache(6)
    B, QL, H, D, H_KV, PAGE, G = 2, 3, 8, 16, 2, 16, 4
    q = rng(7).standard_normal((B, QL, H, D)).astype(np.float16)
    got = O.paged_attention(q, kc, vc, ks, vs, bt, cl, QL)
    for b in range(B):
        L = int(cl[b]); pos = np.arange(L)
        pg, sl = bt[b, pos // PAGE], pos % PAGE
        k = torch.from_numpy(kc[pg, sl].astype(np.float64) * ks[pg, sl][..., None])
        v = torch.from_numpy(vc[pg, sl].astype(np.float64) * vs[pg, sl][..., None])
        k = k.repeat_interleave(G, 1).permute(1, 0, 2)
        v = v.repeat_interleave(G, 1).permute(1, 0, 2)
        qq = torch.from_numpy(q[b].astype(np.float64)).permute(1, 0, 2)
        qpos = L - QL + torch.arange(QL)
        mask = torch.arange(L)[None, :] <= qpos[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(qq, k, v, attn_mask=mask)
        assert np.allclose(got[b], ref.permute(1, 0, 2).numpy(), atol=1e-12, rtol=1e-10)


def test_attention_brute_force_python():
    kc, vc, ks, vs, bt, cl = _small_cache(8, B=1, ctx=(19,), H=2, H_KV=1, D=4)
    q = rng(9).standard_normal((1, 2, 2, 4)).astype(np.float16)
    got = O.paged_attention(q, kc, vc, ks, vs, bt, cl, 2)
    L = 19
    for i in range(2):
        for h in range(2):
            qp = L - 2 + i
            sc = []
            for t in range(qp + 1):
                pg, sl = bt[0, t // 16], t % 16
                sc.append(sum(float(q[0, i, h, d]) * kc[pg, sl, 0, d] * float(ks[pg, sl, 0]) for d in range(4)) / 2.0)
            mx = max(sc); e = [math.exp(x - mx) for x in sc]; den = sum(e)
            for d in range(4):
                o = sum(e[t] / den * vc[bt[0, t // 16], t % 16, 0, d] * float(vs[bt[0, t // 16], t % 16, 0])
                        for t in range(qp + 1))
                assert abs(got[0, i, h, d] - o) < 1e-9


def test_attention_closed_forms():
    kc, vc, ks, vs, bt, cl = _small_cache(10)
    q = rng(11).standard_normal((2, 2, 8, 16)).astype(np.float16)
    vc[:] = 50
    vs[:] = 0.01
    got = O.paged_attention(q, kc, vc, ks, vs, bt, cl, 2)
    assert np.allclose(got[:, :2], 0.5, atol=1e-12)           # constant V -> V
    # single visible key: L = q_len = 1 -> output is that key's scaled value
    kc2, vc2, ks2, vs2, bt2, _ = _small_cache(12, B=1, ctx=(1,))
    one = O.paged_attention(q[:1, :1], kc2, vc2, ks2, vs2, bt2, np.array([1], np.int32), 1)
    expect = vc2[bt2[0, 0], 0].astype(np.float64) * vs2[bt2[0, 0], 0][:, None]
    assert np.allclose(one[0, 0], np.repeat(expect, 4, axis=0), atol=1e-12)


def test_attention_pool_permutation_invariance():
    kc, vc, ks, vs, bt, cl = _small_cache(13)
    q = rng(14).standard_normal((2, 3, 8, 16)).astype(np.float16)
    base = O.paged_attention(q, kc, vc, ks, vs, bt, cl, 3)
    perm = rng(15).permutation(kc.shape[0])
    inv = np.argsort(perm)
    got = O.paged_attention(q, kc[perm], vc[perm], ks[perm], vs[perm], inv[bt].astype(np.int32), cl, 3)
    assert np.array_equal(base, got)


def test_attention_magnitude_closed_forms():
    # mag = sum_t p_t |v_t vs_t|: equals the output when every V entry is >= 0, bounds |out|
    # always, and is the output of the same cache with |V|.
    kc, vc, ks, vs, bt, cl = _small_cache(40)
    q = rng(41).standard_normal((2, 3, 8, 16)).astype(np.float16)
    out, mag = O.paged_attention(q, kc, vc, ks, vs, bt, cl, 3, magnitude=True)
    assert (mag >= np.abs(out) - 1e-12).all()
    absv = np.abs(vc.astype(np.int16)).astype(np.int8)
    pos_out, pos_mag = O.paged_attention(q, kc, absv, ks, vs, bt, cl, 3, magnitude=True)
    assert np.allclose(pos_out, pos_mag, rtol=1e-12, atol=0) and np.allclose(pos_mag, mag, rtol=1e-12, atol=0)
    assert np.array_equal(out, O.paged_attention(q, kc, vc, ks, vs, bt, cl, 3))


def test_silu_mul_matches_torch():
    g = torch.randn(8, 64, generator=torch.Generator().manual_seed(16)).half()
    u = torch.randn(8, 64, generator=torch.Generator().manual_seed(17)).half()
    ref = torch.nn.functional.silu(g.double()) * u.double()
    assert np.allclose(O.silu_mul(g.numpy(), u.numpy()), ref.numpy(), atol=1e-12)


# ---------------------------------------------------------------- paged KV append
def _q8_torch(x):
    """kernels.py:280-283 evaluated with torch's own ops (library round half to even)."""
    s = x.float().abs().amax(-1).clamp(min=1e-8) / 127.0
    return torch.round(x.float() / s[..., None]).clamp(-127, 127).to(torch.int8), s


def test_kv_append_rebuilds_make_paged_kv_cache():
    # Appending every context token of every sequence into an empty cache reproduces the
    # reference generator's cache bit for bit (same generator calls as kernels.py:265-286).
    import kernels as K

    B, ctx, H_KV, D, PAGE, seed = 3, [37, 16, 50], 2, 16, 16, 5
    kc, vc, ks, vs, bt, cl = (t.numpy() for t in K.make_paged_kv(B, ctx, H_KV, D, PAGE, device="cpu", seed=seed))
    g = torch.Generator().manual_seed(seed)
    pages = [(l + PAGE - 1) // PAGE for l in ctx]
    torch.randperm(sum(pages), generator=g)
    kf = torch.randn((sum(pages), PAGE, H_KV, D), generator=g).half().numpy()
    vf = torch.randn((sum(pages), PAGE, H_KV, D), generator=g).half().numpy()
    QL = max(ctx)
    k_new = np.zeros((B, QL, H_KV, D), np.float16)
    v_new = np.zeros((B, QL, H_KV, D), np.float16)
    for b in range(B):
        pos = np.arange(ctx[b])
        k_new[b, :ctx[b]] = kf[bt[b, pos // PAGE], pos % PAGE]
        v_new[b, :ctx[b]] = vf[bt[b, pos // PAGE], pos % PAGE]
    for b in range(B):  # one sequence at a time: q_len = its whole context
        zk, zv = np.zeros_like(kc), np.zeros_like(vc)
        zs, zt = np.zeros_like(ks), np.zeros_like(vs)
        ok, ov, oks, ovs = O.paged_kv_append(k_new[b:b + 1], v_new[b:b + 1], zk, zv, zs, zt, bt[b:b + 1],
                                             cl[b:b + 1], ctx[b])
        pos = np.arange(ctx[b])
        p, s = bt[b, pos // PAGE], pos % PAGE
        assert np.array_equal(ok[p, s], kc[p, s]) and np.array_equal(ov[p, s], vc[p, s])
        assert np.array_equal(oks[p, s].view(np.uint16), ks[p, s].view(np.uint16))
        assert np.array_equal(ovs[p, s].view(np.uint16), vs[p, s].view(np.uint16))


def test_kv_append_kats_and_torch_rounding():
    # amax 127 gives s = 1 exactly: x / s = x, so 2.5 -> 2 and -3.5 -> -4 (half to even).
    row = np.zeros(16, np.float16)
    row[:5] = [127.0, 2.5, -3.5, 0.5, -127.0]
    k_new = np.zeros((1, 1, 1, 16), np.float16)
    k_new[0, 0, 0] = row
    kc = np.zeros((2, 16, 1, 16), np.int8)
    ks = np.zeros((2, 16, 1), np.float32)
    bt = np.array([[1]], np.int32)
    cl = np.array([4], np.int32)  # the new token sits at position 3 of page 1
    ok, _, oks, _ = O.paged_kv_append(k_new, k_new, kc, kc, ks, ks, bt, cl, 1)
    assert list(ok[1, 3, 0, :5]) == [127, 2, -4, 0, -127] and oks[1, 3, 0] == 1.0
    assert (ok[0] == 0).all() and (ok[1, :3] == 0).all() and (ok[1, 4:] == 0).all()
    # all-zero row: the 1e-8 clamp gives s = 1e-8 / 127 and q = 0
    zero = np.zeros_like(k_new)
    ok, _, oks, _ = O.paged_kv_append(zero, zero, kc, kc, ks, ks, bt, cl, 1)
    assert (ok == 0).all() and oks[1, 3, 0] == np.float32(np.float32(1e-8) / np.float32(127))
    # random rows against torch's own round/clamp
    r = rng(9)
    x = (r.standard_normal((2, 3, 2, 64)) * 3).astype(np.float16)
    kc = np.zeros((4, 16, 2, 64), np.int8)
    ks = np.zeros((4, 16, 2), np.float16)
    bt = np.array([[2, 0], [3, 1]], np.int32)
    cl = np.array([18, 3], np.int32)
    ok, _, oks, _ = O.paged_kv_append(x, x, kc, kc, ks, ks, bt, cl, 3)
    tq, ts = _q8_torch(torch.from_numpy(x))
    for b, (p, s0) in enumerate([(0, 15), (3, 0)]):
        pos = cl[b] - 3 + np.arange(3)
        pages, slots = bt[b, pos // 16], pos % 16
        assert np.array_equal(ok[pages, slots], tq[b].numpy())
        assert np.array_equal(oks[pages, slots].view(np.uint16), ts[b].half().numpy().view(np.uint16))


def test_kv_append_skips_rows_outside_the_cache():
    x = np.ones((2, 2, 1, 16), np.float16)
    kc = np.full((2, 16, 1, 16), 7, np.int8)
    ks = np.full((2, 16, 1), 3.0, np.float16)
    bt = np.array([[0], [5]], np.int32)      # sequence 1 names a page outside the pool
    cl = np.array([17, 2], np.int32)         # sequence 0's second token falls past max_pages
    ok, _, oks, _ = O.paged_kv_append(x, x, kc, kc, ks, ks, bt, cl, 2)
    assert (ok[0, 15] == 127).all() and (ok[0, :15] == 7).all() and (ok[1] == 7).all()
    assert oks[0, 15, 0] == np.float16(1.0 / 127.0) and (oks[1] == 3.0).all()


# ---------------------------------------------------------------- W4A8
def test_w4a8_brute_force_and_kats():
    r = rng(21)
    a = r.integers(-127, 128, (3, 10), dtype=np.int8)
    qu = r.integers(0, 16, (4, 10)).astype(np.uint8)
    sa = r.uniform(0.005, 0.02, 3).astype(np.float32)
    sw = r.uniform(0.001, 0.01, 4).astype(np.float32)
    got = O.w4a8(a, sa, qu, sw)
    for m in range(3):
        for n in range(4):
            acc = sum(int(a[m, k]) * (int(qu[n, k]) - 8) for k in range(10))
            want = np.float16(np.float32(np.float32(np.float32(acc) * sa[m]) * sw[n]))
            assert got[m, n].view(np.uint16) == want.view(np.uint16)
    # nibble 8 is weight 0; nibble 0 is -8; nibble 15 is +7
    ones = np.ones((1, 64), np.int8)
    s1 = np.ones(1, np.float32)
    assert O.w4a8(ones, s1, np.full((1, 64), 8, np.uint8), s1)[0, 0] == 0
    assert O.w4a8(ones, s1, np.zeros((1, 64), np.uint8), s1)[0, 0] == -512
    assert O.w4a8(ones, s1, np.full((1, 64), 15, np.uint8), s1)[0, 0] == 448


def test_w4a8_channel_quantizer_matches_torch_restatement():
    import kernels as K

    r = rng(22)
    w = (r.standard_normal((24, 256)) * 0.05).astype(np.float32)
    w[3, :] = 0.0                              # the 1e-8 clamp
    w[5, :4] = [7.0, 3.5, -2.5, 0.5]           # amax 7 -> sc 1: half to even on 3.5, -2.5, 0.5
    w[5, 4:] = 0.0
    qu, sc = O.quantize_weight_int4_channel(w)
    assert list(qu[5, :4].astype(int) - 8) == [7, 4, -2, 0] and sc[5] == 1.0
    assert (qu[3] == 8).all() and sc[3] == np.float32(np.float32(1e-8) / np.float32(7))
    packed, tsc = K.quantize_weight_int4_channel(torch.from_numpy(w))
    assert np.array_equal(O.unpack_int4_u8(packed.numpy()), qu)
    assert np.array_equal(tsc.numpy().view(np.uint32), sc.view(np.uint32))


# ---------------------------------------------------------------- CPU baseline formulas
def test_cpu_baseline_w8a8_int_mm_is_bitexact():
    from oracle import cpu_baseline as C
    r = rng(30)
    a = r.integers(-127, 128, (20, 4096), dtype=np.int8)
    w = r.integers(-127, 128, (48, 4096), dtype=np.int8)
    sa = r.uniform(0.005, 0.02, 20).astype(np.float32)
    sw = r.uniform(0.001, 0.01, 48).astype(np.float32)
    got = C.w8a8_int_mm(torch.from_numpy(a), torch.from_numpy(sa), torch.from_numpy(w).T.contiguous(),
                        torch.from_numpy(sw)).numpy()
    assert np.array_equal(got.view(np.uint16), O.w8a8(a, sa, w, sw).view(np.uint16))


def test_cpu_baseline_fp32_formula_exact_below_2_24():
    # With 127 * 127 * K < 2**24 every fp32 partial sum is exact, so the reference test's float
    # formula equals the kernel's fp32 epilogue value and rounds to the same fp16.
    from oracle import cpu_baseline as C
    r = rng(31)
    K = 1040
    assert 127 * 127 * K < 2 ** 24
    a = np.full((3, K), 127, np.int8); a[1] = -127; a[2] = r.integers(-127, 128, K, dtype=np.int8)
    w = r.integers(-127, 128, (40, K), dtype=np.int8); w[0] = 127
    sa = r.uniform(0.005, 0.02, 3).astype(np.float32)
    sw = r.uniform(0.001, 0.01, 40).astype(np.float32)
    got = C.w8a8_fp32_formula(torch.from_numpy(a), torch.from_numpy(sa), torch.from_numpy(w), torch.from_numpy(sw))
    assert np.array_equal(got.half().numpy().view(np.uint16), O.w8a8(a, sa, w, sw).view(np.uint16))


def test_cpu_baseline_w4a16_and_attention_match_oracle():
    from oracle import cpu_baseline as C
    r = rng(32)
    N, K, G = 64, 512, 128
    qu = r.integers(0, 16, (N, K)).astype(np.uint8)
    sc = r.uniform(0.002, 0.02, (N, K // G)).astype(np.float16)
    x = r.standard_normal((9, K)).astype(np.float16)
    deq = O.dequant_int4(qu, sc, G)
    got = C.w4a16_fp32(torch.from_numpy(x), torch.from_numpy(deq)).float().numpy()
    ref = O.w4a16(x, qu, sc, G)
    assert np.abs(got - ref).max() <= 2e-3 * np.abs(ref).max()
    zero = C.w4a16_fp32(torch.from_numpy(x), torch.zeros((N, K), dtype=torch.float16))
    assert (zero == 0).all()
    kc, vc, ks, vs, bt, cl = _small_cache(33, B=2, ctx=(45, 19), H=8, H_KV=2, D=32)
    q = rng(34).standard_normal((2, 4, 8, 32)).astype(np.float16)
    got = C.paged_attention_fp32(*(torch.from_numpy(t) for t in (q, kc, vc, ks, vs, bt, cl)), 3).float().numpy()
    ref = O.paged_attention(q, kc, vc, ks, vs, bt, cl, 3)
    assert np.abs(got[:, :3] - ref[:, :3]).max() < 2e-3 and (got[:, 3:] == 0).all()
