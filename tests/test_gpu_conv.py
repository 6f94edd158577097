"""pk_conv_step (GLU -> pad mask -> causal depthwise conv with the per-stream
cache -> LayerNorm -> SiLU, cache updated in place) on the GPU against the oracle
(oracle/conv.py, pinned in test_oracle_conv.py).

Bars:
* outputs: |got - ref| <= atol + rtol * |ref| against float64 on the same
  dtype-rounded inputs, (atol, rtol) = (1e-5, 1e-5) fp32, (1e-3, 2^-10) fp16,
  (8e-3, 2^-7) bf16 -- the output is rounded to the storage dtype once;
* cache rows carried over from the previous cache: bit-exact;
* cache rows holding this step's frames (GLU outputs rounded to the dtype):
  within one unit of the dtype's last place of the oracle's rounded value
  (eight for fp32, where the GLU's exp differs in the last bits);
* every slot outside the batch and every other layer: bit-exact, untouched."""

import numpy as np
import pytest
import torch

from oracle import conv as oc
from parakeet_amd import ops

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
TOL = {torch.float32: (1e-5, 1e-5), torch.float16: (1e-3, 2.0**-10), torch.bfloat16: (8e-3, 2.0**-7)}
CACHE_REL = {torch.float32: 8 * 2.0**-23, torch.float16: 2.0**-10, torch.bfloat16: 2.0**-7}


def _params(D, K, dt, seed, bias):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(D, 1, K, generator=g) / K**0.5
    b = torch.randn(D, generator=g) * 0.1 if bias else None
    lw = 1.0 + 0.1 * torch.randn(D, generator=g)
    lb = 0.1 * torch.randn(D, generator=g)
    return tuple(None if x is None else x.to(dt) for x in (w, b, lw, lb))


def _f64(t):
    return None if t is None else t.detach().double().cpu().numpy()


def _close(got, ref, dt, what):
    atol, rtol = TOL[dt]
    err = np.abs(got - ref)
    lim = atol + rtol * np.abs(ref)
    assert (err <= lim).all(), f"{what}: max excess {(err - lim).max():.3e}, max err {err.max():.3e}"


def _cache_close(got, ref, dt, what):
    err = np.abs(got - ref)
    lim = CACHE_REL[dt] * np.abs(ref) + 2.0**-24
    assert (err <= lim).all(), f"{what}: cache frame off by {(err - lim).max():.3e} beyond one ulp"


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize(
    "D,T,K,bias",
    [(512, 2, 9, False), (1024, 2, 9, False), (256, 14, 9, True), (64, 1, 3, True), (136, 5, 5, False)],
)
def test_conv_step_matches_oracle(cuda, dt, D, T, K, bias):
    if dt == torch.float32 and D % 4 or dt != torch.float32 and D % 8:
        pytest.skip("d_model not a whole number of 16-byte chunks")
    S, Ly, B, layer, steps = 12, 3, 7, 1, 4
    rng = np.random.default_rng(D * 31 + T * 7 + K)
    slots = rng.permutation(S)[:B].astype(np.int32)
    slots_t = torch.from_numpy(slots).to(cuda)
    w, b, lw, lb = _params(D, K, dt, seed=D + K, bias=bias)
    wd, bd, lwd, lbd = (None if x is None else x.to(cuda) for x in (w, b, lw, lb))
    g = torch.Generator().manual_seed(K)
    cache = torch.randn(S, Ly, K - 1, D, generator=g).to(dt).to(cuda)
    for step in range(steps):
        h = torch.randn(B, T, 2 * D, generator=g).to(dt)
        pad = torch.from_numpy(rng.random((B, T)) < (0.3 if step == 2 else 0.0))
        before = cache.clone()
        y = ops.conv_step(h.to(cuda), cache, wd, lwd, lbd, layer=layer, slots=slots_t, pad_mask=pad.to(cuda), dw_bias=bd)
        torch.cuda.synchronize()
        prev = _f64(before[slots_t.long(), layer])
        ref_y, ref_c = oc.conv_module_step(
            _f64(h), prev, pad.numpy(), _f64(w).reshape(D, K), _f64(b), _f64(lw), _f64(lb), 1e-5, store_dtype=dt
        )
        _close(_f64(y), ref_y, dt, f"step {step} output")
        new = _f64(cache[slots_t.long(), layer])
        keep = max(K - 1 - T, 0)
        np.testing.assert_array_equal(new[:, :keep], prev[:, T : T + keep], err_msg=f"step {step}: carried rows")
        _cache_close(new[:, keep:], ref_c[:, keep:], dt, f"step {step}")
        # everything outside (slots[b], layer) is untouched
        other = torch.ones(S, Ly, dtype=torch.bool)
        other[torch.from_numpy(slots).long(), layer] = False
        assert torch.equal(cache[other.to(cuda)], before[other.to(cuda)])


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_padding_sources_agree(cuda, dt):
    """pad_mask, per-stream lengths and one scalar length describe the same
    padding (encoder.py:204-205 builds pad_mask from lengths)."""
    S, Ly, B, T, D, K = 6, 2, 6, 4, 512, 9
    w, _, lw, lb = (x.to(cuda) if x is not None else None for x in _params(D, K, dt, 3, False))
    g = torch.Generator().manual_seed(9)
    h = torch.randn(B, T, 2 * D, generator=g).to(dt).to(cuda)
    base = torch.randn(S, Ly, K - 1, D, generator=g).to(dt).to(cuda)
    lengths = torch.tensor([4, 3, 2, 1, 0, 4], dtype=torch.int64, device=cuda)
    pad = torch.arange(T, device=cuda)[None, :] >= lengths[:, None]
    c1, c2 = base.clone(), base.clone()
    y1 = ops.conv_step(h, c1, w, lw, lb, pad_mask=pad)
    y2 = ops.conv_step(h, c2, w, lw, lb, lengths=lengths)
    assert torch.equal(y1, y2) and torch.equal(c1, c2)
    c3, c4 = base.clone(), base.clone()
    y3 = ops.conv_step(h, c3, w, lw, lb, lengths=2)
    y4 = ops.conv_step(h, c4, w, lw, lb, pad_mask=torch.arange(T, device=cuda)[None, :].expand(B, T) >= 2)
    assert torch.equal(y3, y4) and torch.equal(c3, c4)


def test_stream_of_steps_equals_one_shot(cuda):
    """128 streams x 60 steps of 2 frames (the small model's shape, fp16) fed
    through the cache give the frames and the final cache of one causal pass over
    all 120 frames from a zero cache (cache.py:30-34)."""
    dt, B, D, K, T, steps = torch.float16, 128, 512, 9, 2, 60
    w, _, lw, lb = _params(D, K, dt, 21, False)
    g = torch.Generator().manual_seed(22)
    h = torch.randn(B, steps * T, 2 * D, generator=g).to(dt)
    cache = torch.zeros(B, 1, K - 1, D, dtype=dt, device=cuda)
    hd, wd, lwd, lbd = h.to(cuda), w.to(cuda), lw.to(cuda), lb.to(cuda)
    ys = [ops.conv_step(hd[:, s * T : (s + 1) * T], cache, wd, lwd, lbd) for s in range(steps)]
    torch.cuda.synchronize()
    ref_y, ref_c = oc.conv_module_step(
        _f64(h), np.zeros((B, K - 1, D)), None, _f64(w).reshape(D, K), None, _f64(lw), _f64(lb), 1e-5, store_dtype=dt
    )
    _close(_f64(torch.cat(ys, dim=1)), ref_y, dt, "streamed outputs")
    _cache_close(_f64(cache[:, 0]), ref_c, dt, "final cache")


def test_empty_batch_is_a_no_op(cuda):
    cache = torch.zeros(2, 1, 8, 512, dtype=torch.float16, device=cuda)
    w, _, lw, lb = (x.to(cuda) if x is not None else None for x in _params(512, 9, torch.float16, 1, False))
    y = ops.conv_step(torch.empty(0, 2, 1024, dtype=torch.float16, device=cuda), cache, w, lw, lb)
    assert y.shape == (0, 2, 512)
    assert not cache.any()


@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_module_in_place_and_tensor_state_agree(cuda, dt):
    """ConformerConvolution.forward (convolution.py:150-162) through the paged
    ModelCache (state updated in place per slot) and through the reference's
    tensor state (get_conv_cache -> forward -> update_conv_cache, cache.py:47-53)
    give identical frames and states, both matching the oracle with the module's
    own pointwise projections in float64."""
    from parakeet_amd.modules.cache import ModelCache
    from parakeet_amd.modules.encoder import ConformerConvolution

    D, K, N, Ly, layer = 256, 9, 6, 2, 1
    torch.manual_seed(5)
    conv = ConformerConvolution(D, K).to(dt).to(cuda)
    with torch.no_grad():
        conv.batch_norm.weight.uniform_(0.5, 1.5)
        conv.batch_norm.bias.uniform_(-0.2, 0.2)
    a = ModelCache(Ly, (70, 1), D, K, batch_size=N, device=cuda, dtype=dt)
    b = ModelCache(Ly, (70, 1), D, K, batch_size=N, device=cuda, dtype=dt)
    slots = [4, 1, 3]
    va, vb = a.batch(slots), b.batch(slots)
    g = torch.Generator().manual_seed(6)
    for step in range(5):
        x = torch.randn(len(slots), 2, D, generator=g).to(dt).to(cuda)
        pad = torch.zeros(len(slots), 2, dtype=torch.bool, device=cuda)
        prev = vb.get_conv_cache(layer).double().cpu().numpy()  # [B, D, K-1]
        with torch.no_grad():
            ya, sa = conv(x, pad, cache=va.conv_ref(layer))
            va.update_conv_cache(layer, sa)
            yb, sb = conv(x, pad, cache=vb.get_conv_cache(layer))
            vb.update_conv_cache(layer, sb)
        assert sa is None and tuple(sb.shape) == (len(slots), D, K - 1)
        assert torch.equal(ya, yb)
        assert torch.equal(a.conv_frames, b.conv_frames)
        w2 = _f64(conv.pointwise_conv2.weight.squeeze(-1))
        # the oracle takes the projection output the module computed (the GEMM is torch's)
        with torch.no_grad():
            h = _f64(torch.nn.functional.linear(x, conv.pointwise_conv1.weight.squeeze(-1)))
        ry, rc = oc.conv_module_step(
            h, prev.transpose(0, 2, 1), None, _f64(conv.depthwise_conv.weight).reshape(D, K), None,
            _f64(conv.batch_norm.weight), _f64(conv.batch_norm.bias), conv.batch_norm.eps, store_dtype=dt,
        )
        # the pointwise projection after the step rounds once more: (atol, rtol)
        # = (1e-5, 1e-5) fp32, (4e-3, 2^-9) fp16 on the module output
        atol, rtol = (1e-5, 1e-5) if dt == torch.float32 else (4e-3, 2.0**-9)
        ref_out = oc.round_to(ry, dt) @ w2.T
        err = np.abs(_f64(ya) - ref_out)
        assert (err <= atol + rtol * np.abs(ref_out)).all(), f"step {step}: module output err {err.max():.3e}"
        _cache_close(_f64(va.get_conv_cache(layer)).transpose(0, 2, 1), rc, dt, f"step {step} module state")
    # slots outside the batch never moved; reset_slot empties one slot's state
    assert not a.conv_frames[[0, 2, 5]].any()
    a.reset_slot(4)
    assert not a.conv_frames[4].any() and a.conv_frames[1].any()
    assert tuple(a.conv.shape) == (N, Ly, D, K - 1)


@pytest.mark.parametrize("B,L,D,T,dt,blk", [(2048, 13, 512, 2, torch.float16, 256), (600, 24, 1024, 14, torch.bfloat16, 64)],
                         ids=["frame-by-frame", "frames-in-parallel"])
def test_streaming_policy_is_bit_exact(cuda, B, L, D, T, dt, blk):
    """A batch whose conv caches over all layers pass the host's 192 MiB
    streaming threshold (2048 streams x 13 layers x 8 rows x 512 x 2 bytes =
    218 MB at 2 frames; 600 x 24 x 8 x 1024 x 2 = 236 MB at 14 frames, where
    both batches take the frames-in-parallel kernel) runs with the streaming
    cache policy; the same streams in blocks (27 MB, 25 MB) run with the
    cached one.  Outputs and updated caches must agree bit for bit."""
    K, layer = 9, 5
    w, _, lw, lb = _params(D, K, dt, 11, False)
    wd, lwd, lbd = w.to(cuda), lw.to(cuda), lb.to(cuda)
    g = torch.Generator().manual_seed(12)
    h = torch.randn(B, T, 2 * D, generator=g).to(dt).to(cuda)
    c1 = torch.randn(B, L, K - 1, D, generator=g).to(dt).to(cuda)
    c2 = c1.clone()
    y1 = ops.conv_step(h, c1, wd, lwd, lbd, layer=layer)
    y2 = torch.empty_like(y1)
    for b0 in range(0, B, blk):
        b1 = min(B, b0 + blk)
        slots = torch.arange(b0, b1, dtype=torch.int32, device=cuda)
        y2[b0:b1] = ops.conv_step(h[b0:b1], c2, wd, lwd, lbd, layer=layer, slots=slots)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    assert torch.equal(c1.view(torch.int16), c2.view(torch.int16))


def _bits(t):
    return t.view(torch.int32) if t.element_size() == 4 else t.view(torch.int16)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("D,T,K", [(1024, 14, 9), (520, 7, 9), (136, 5, 5), (24, 3, 9), (512, 14, 3)])
def test_chunk_form_equals_two_frame_steps(cuda, dt, D, T, K):
    """A chunk of 3 or more frames goes to the frames-in-parallel kernel (the
    window staged in LDS, groups of waves over the frames) at batches under
    about six of the other kernel's waves a CU; chunks of 1-2 frames to the
    frame-by-frame one.  The same frames fed as one T-frame step
    and as steps of 2 (and a last 1) through the cache give the same outputs
    and the same final cache, bit for bit: every sum is the same in the same
    order, for d_model a power of two or not (where 1/d_model is inexact and a
    fused and an unfused rounding of the LayerNorm statistics would differ)."""
    if dt == torch.float32 and D % 4 or dt != torch.float32 and D % 8:
        pytest.skip("d_model not a whole number of 16-byte chunks")
    print(f"\n[conv chunk form] {dt} D={D} T={T} K={K}", flush=True)
    S, Ly, B, layer = 9, 2, 7, 1
    rng = np.random.default_rng(D + T + K)
    slots = torch.from_numpy(rng.permutation(S)[:B].astype(np.int32)).to(cuda)
    w, b, lw, lb = (None if x is None else x.to(cuda) for x in _params(D, K, dt, seed=D * 3 + K, bias=True))
    g = torch.Generator().manual_seed(T * 5 + K)
    c1 = torch.randn(S, Ly, K - 1, D, generator=g).to(dt).to(cuda)
    c2 = c1.clone()
    h = torch.randn(B, T, 2 * D, generator=g).to(dt).to(cuda)
    pad = torch.from_numpy(rng.random((B, T)) < 0.25).to(cuda)
    y1 = ops.conv_step(h, c1, w, lw, lb, layer=layer, slots=slots, pad_mask=pad, dw_bias=b)
    parts = []
    for t0 in range(0, T, 2):
        t1 = min(T, t0 + 2)
        parts.append(ops.conv_step(h[:, t0:t1].contiguous(), c2, w, lw, lb, layer=layer, slots=slots,
                                   pad_mask=pad[:, t0:t1].contiguous(), dw_bias=b))
    torch.cuda.synchronize()
    y2 = torch.cat(parts, dim=1)
    assert torch.equal(_bits(y1), _bits(y2)), f"outputs differ at {int((_bits(y1) != _bits(y2)).sum())} values"
    assert torch.equal(_bits(c1), _bits(c2)), "caches differ"
