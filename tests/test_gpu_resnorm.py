"""pk_residual_norm against torch: a Conformer layer's residual update and the
LayerNorm that reads it (parakeet/modules/encoder.py:61-80).

The residual is exact arithmetic on stored values: torch's own
``residual + branch * alpha`` in the model dtype (``branch * alpha`` rounded,
then the sum rounded) must come out bit for bit.  The norm is compared with a
float32 LayerNorm of that residual (the plain fp32 reference of the op),
rounded to the dtype: within one rounding of the dtype (relative 2^-10 fp16,
2^-7 bf16; 1e-5 fp32 for the statistics' summation order), and with torch's own
LayerNorm in the dtype to the same bar."""

import pytest
import torch
import torch.nn.functional as F

from parakeet_amd import ops

REL = {torch.float32: 1e-5, torch.float16: 2.0**-10, torch.bfloat16: 2.0**-7}
ABS = {torch.float32: 1e-5, torch.float16: 2.0**-12, torch.bfloat16: 2.0**-9}


def _case(cuda, dtype, rows, D, alpha, in_place, seed):
    print(f"\n[resnorm] dtype={dtype} rows={rows} D={D} alpha={alpha} in_place={in_place}", flush=True)
    g = torch.Generator().manual_seed(seed)
    res = (3.0 * torch.randn(rows, D, generator=g) + 0.5).to(dtype).to(cuda)
    br = torch.randn(rows, D, generator=g).to(dtype).to(cuda)
    w = (1.0 + 0.2 * torch.randn(D, generator=g)).to(dtype).to(cuda)
    b = (0.2 * torch.randn(D, generator=g)).to(dtype).to(cuda)
    want_r = res + br * alpha if alpha != 1.0 else res + br
    ref = F.layer_norm(want_r.float(), (D,), w.float(), b.float(), 1e-5).to(dtype).float()
    native = F.layer_norm(want_r, (D,), w, b, 1e-5).float()
    before = res.clone()
    r, n = ops.residual_norm(res, br, w, b, alpha=alpha, eps=1e-5, in_place=in_place)
    torch.cuda.synchronize()
    assert torch.equal(r, want_r), float((r.float() - want_r.float()).abs().max())
    if in_place:
        assert r.data_ptr() == res.data_ptr()
    else:
        assert torch.equal(res, before)  # the input is not modified
    got = n.float()
    bar = REL[dtype] * ref.abs() + ABS[dtype]
    err = (got - ref).abs()
    print(f"  max err vs fp32 LayerNorm {float(err.max()):.3e}, vs torch {dtype}: "
          f"{float((got - native).abs().max()):.3e}", flush=True)
    assert bool((err <= bar).all()), float((err - bar).max())
    assert bool(((got - native).abs() <= REL[dtype] * native.abs() + ABS[dtype]).all())


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [512, 1024, 176])
@pytest.mark.parametrize("alpha", [1.0, 0.5])
def test_residual_norm_matches_torch(cuda, dtype, D, alpha):
    _case(cuda, dtype, rows=257, D=D, alpha=alpha, in_place=False, seed=D + int(alpha * 10))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_residual_norm_in_place_and_edge_rows(cuda, dtype):
    _case(cuda, dtype, rows=1, D=512, alpha=0.5, in_place=True, seed=1)
    _case(cuda, dtype, rows=5, D=4096 if dtype != torch.float32 else 2048, alpha=1.0, in_place=True, seed=2)
    _case(cuda, dtype, rows=1792, D=1024, alpha=0.5, in_place=True, seed=3)


@pytest.mark.gpu
def test_residual_norm_three_dims_and_empty(cuda):
    g = torch.Generator().manual_seed(4)
    res = torch.randn(3, 2, 512, generator=g).half().to(cuda)
    br = torch.randn(3, 2, 512, generator=g).half().to(cuda)
    w = torch.ones(512, dtype=torch.float16, device=cuda)
    b = torch.zeros(512, dtype=torch.float16, device=cuda)
    r, n = ops.residual_norm(res, br, w, b, alpha=0.5)
    assert r.shape == (3, 2, 512) and torch.equal(r, res + br * 0.5)
    ref = F.layer_norm((res + br * 0.5).float(), (512,)).half().float()
    assert float((n.float() - ref).abs().max()) <= 2.0**-10 * float(ref.abs().max()) + 2.0**-12
    e = torch.empty(0, 512, dtype=torch.float16, device=cuda)
    r0, n0 = ops.residual_norm(e, e, w, b)
    assert r0.shape == (0, 512) and n0.shape == (0, 512)
