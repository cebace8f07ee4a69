"""Device-side layer steps: per-token INT8 quantisation (bit-exact with the reference
formula, kernels.py:58-62), SiLU*mul (within one fp16 ulp of the float64 closed form),
and their fusion (bit-identical to running the two steps)."""
import numpy as np
import pytest
import torch

import kernels as K
from gpu_util import note
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("shape", [(1, 7), (37, 4096), (288, 14336)])
def test_quantize_act_int8_gpu_bit_exact(shape):
    note(f"quantize_act_int8 {shape}")
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(shape[1])).half() * 3
    x[0, 0] = 0.0
    q, s = K.quantize_act_int8_gpu(x.to(DEV))
    torch.cuda.synchronize()
    qo, so = O.quantize_rows_int8(x.numpy())
    assert np.array_equal(q.cpu().numpy(), qo) and np.array_equal(s.cpu().numpy(), so)
    qz, sz = K.quantize_act_int8_gpu(torch.zeros(3, 64, dtype=torch.float16, device=DEV))
    torch.cuda.synchronize()
    assert bool((qz == 0).all()) and np.array_equal(sz.cpu().numpy(), np.full(3, np.float32(1e-8) / np.float32(127)))


@pytest.mark.parametrize("shape", [(96, 14336), (7, 1001), (3, 40000), (5, 8)])
def test_silu_mul_and_fused_quant(shape):
    # Register-resident vector path (rows of 8-element multiples up to 32768) and the
    # element-wise fallback (odd widths, wider rows).
    note(f"silu_mul + fused quant {shape}")
    g = torch.randn(*shape, generator=torch.Generator().manual_seed(1)).half() * 4
    u = torch.randn(*shape, generator=torch.Generator().manual_seed(2)).half()
    gd, ud = g.to(DEV), u.to(DEV)
    h = K.silu_mul(gd, ud)
    q, s = K.silu_mul_quant_int8(gd, ud)
    q2, s2 = K.quantize_act_int8_gpu(h)
    torch.cuda.synchronize()
    ref = O.silu_mul(g.numpy(), u.numpy())
    hf = h.float().cpu().numpy().astype(np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert (np.abs(hf - ref) <= ulp + 1e-7).all()
    assert torch.equal(q, q2) and torch.equal(s, s2)


def test_elementwise_plan_rows():
    note("elementwise plan rows")
    g = torch.randn(64, 256, device=DEV).half()
    u = torch.randn(64, 256, device=DEV).half()
    plan = torch.zeros(8, dtype=torch.int32, device=DEV)
    plan[0] = 10
    q = torch.full((64, 256), 5, dtype=torch.int8, device=DEV)
    s = torch.full((64,), 9.0, device=DEV)
    K.silu_mul_quant_int8(g, u, q=q, s=s, plan=plan, grid_m_max=64)
    qe, se = K.silu_mul_quant_int8(g[:10], u[:10])
    torch.cuda.synchronize()
    assert torch.equal(q[:10], qe) and torch.equal(s[:10], se)
    assert bool((q[10:] == 5).all()) and bool((s[10:] == 9.0).all())
