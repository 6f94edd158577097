"""Pins oracle/encoder.py, the float64 restatement of one streaming
ConformerEncoder step (parakeet/modules/encoder.py:11-81,229-267):

* against the drop-in module tree run in float64 on the CPU with the oracle's
  attention, conv step and masks (tests/_dense_encoder.py): a second, separately
  written composition of the layer (residuals, 0.5 feed-forward scales, the
  five LayerNorms, biases) and of the state advance, step after step through
  eviction, with and without biases;
* a closed form: with the feed-forward, attention and conv outputs zeroed, each
  layer is LayerNorm(x), checked against torch's layer_norm;
* a case computed by hand from encoder.py:50-81 (the numbers are in the test):
  the feed-forward branches made silu and 3 silu, attention and conv outputs
  zeroed, so the residual order, the two 0.5 scales and the norm placement
  fix the output;
* a planted mistake (a feed-forward branch without its 0.5 scale) is caught.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import encoder as oe
from oracle import relpos
from parakeet_amd.modules.cache import StreamingState
from parakeet_amd.modules.encoder import ConformerEncoder

from _dense_encoder import DenseCache, init_attention, module_reference


def _encoder(D, H, Ly, left, right, K, bias, seed):
    torch.manual_seed(seed)
    enc = ConformerEncoder(
        feat_in=80, hidden_size=D, ff_expansion_factor=2, num_layers=Ly, num_heads=H, subsampling_factor=8,
        pos_emb_max_len=64, conv_kernel_size=K, att_context_size=[left, right], subsampling_conv_channels=16,
        use_bias=bias,
    )
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for layer in enc.layers:
            init_attention(layer.self_attn, D, seed=seed + 10 + layer.layer_idx)
            for mod in layer.modules():
                if isinstance(mod, torch.nn.LayerNorm):  # off the identity, so a swapped norm shows
                    mod.weight.copy_(1.0 + 0.2 * torch.randn(mod.weight.shape, generator=g))
                    mod.bias.copy_(0.2 * torch.randn(mod.bias.shape, generator=g))
                if isinstance(mod, (torch.nn.Linear, torch.nn.Conv1d)) and mod.bias is not None:
                    mod.bias.copy_(0.1 * torch.randn(mod.bias.shape, generator=g))
    return enc.double()


def _state_dict(enc):
    return {k: v.detach().double().numpy() for k, v in enc.state_dict().items()}


def _run_both(enc, B, steps, seed, zero_len_stream=False):
    left, right = enc.att_context_size
    T = right + 1
    Ly, D, K = len(enc.layers), enc.embed_dim, enc.conv_kernel_size
    H = enc.layers[0].self_attn.num_heads
    ref = module_reference(enc, H)
    dense = DenseCache(B, Ly, left, right, D, K)
    st = oe.EncoderState(B, Ly, left, right, D, K)
    sd = _state_dict(enc)
    # the table is fp32 on both sides (attention.py:36-45); an ulp of difference
    # between libraries' fp32 exp of a frequency moves the angle at position p by
    # about p * 2^-24 relative: up to 1e-6 in the table, 3e-8 in the outputs here
    pe = relpos.sinusoid_table(64, D).astype(np.float64)
    proc = torch.zeros(B, dtype=torch.int64)
    cl = torch.zeros(B, dtype=torch.int64)
    g = torch.Generator().manual_seed(seed)
    worst = 0.0
    outs = []
    for step in range(steps):
        x = torch.randn(B, T, D, generator=g, dtype=torch.float64)
        length = torch.full((B,), T, dtype=torch.int64)
        if zero_len_stream:
            length[0] = 1  # a short chunk: one valid frame, one padded
        with torch.no_grad():
            rout, _ = ref(x.clone(), StreamingState(dense, proc, cl), length=length)
        got = oe.encoder_step(x.numpy(), sd, st, length.numpy(), Ly, H, pe)
        worst = max(worst, float(np.abs(got - rout.numpy()).max()))
        outs.append(got)
        assert st.processed.tolist() == proc.tolist()
        assert st.cache_len.tolist() == cl.tolist()
    return worst, outs


@pytest.mark.parametrize("bias", [False, True])
def test_oracle_encoder_matches_module_composition(bias):
    enc = _encoder(D=32, H=4, Ly=2, left=6, right=1, K=5, bias=bias, seed=3)
    worst, _ = _run_both(enc, B=3, steps=9, seed=4)  # the window fills after 3 steps
    assert worst < 1e-6, worst


def test_oracle_encoder_short_chunk_and_wider_chunk():
    enc = _encoder(D=32, H=2, Ly=1, left=8, right=3, K=3, bias=False, seed=5)
    worst, _ = _run_both(enc, B=2, steps=6, seed=6, zero_len_stream=True)
    assert worst < 1e-6, worst


def test_zero_branches_leave_the_layer_norms():
    """Feed-forward linear2, linear_out and pointwise_conv2 zeroed: every layer
    returns norm_out(x) of its input."""
    enc = _encoder(D=32, H=4, Ly=2, left=6, right=1, K=5, bias=False, seed=7)
    with torch.no_grad():
        for layer in enc.layers:
            layer.feed_forward1.linear2.weight.zero_()
            layer.feed_forward2.linear2.weight.zero_()
            layer.self_attn.linear_out.weight.zero_()
            layer.conv.pointwise_conv2.weight.zero_()
    sd = _state_dict(enc)
    st = oe.EncoderState(2, 2, 6, 1, 32, 5)
    x = torch.randn(2, 2, 32, generator=torch.Generator().manual_seed(8), dtype=torch.float64)
    got = oe.encoder_step(x.numpy(), sd, st, np.full(2, 2), 2, 4, relpos.sinusoid_table(64, 32).astype(np.float64))
    want = x
    for layer in enc.layers:
        want = F.layer_norm(want, (32,), layer.norm_out.weight, layer.norm_out.bias, 1e-5)
    np.testing.assert_allclose(got, want.detach().transpose(1, 2).numpy(), atol=1e-12)


def test_planted_unscaled_feed_forward_is_caught(monkeypatch):
    enc = _encoder(D=32, H=4, Ly=2, left=6, right=1, K=5, bias=False, seed=9)
    _, good = _run_both(enc, B=2, steps=2, seed=10)
    real = oe.feed_forward
    monkeypatch.setattr(oe, "feed_forward", lambda x, sd, prefix: 2.0 * real(x, sd, prefix))
    worst, _ = _run_both(enc, B=2, steps=2, seed=10)
    assert worst > 1e-2, worst


def test_layer_composition_by_hand():
    """One layer, d_model 4 (2 heads), unit LayerNorms, computed by hand from
    ConformerLayer.forward (encoder.py:50-81):
      FF1(y) = linear2(silu(linear1(y))) with linear1 = [I; 0], linear2 = [I, 0]: silu(y)
      FF2 the same with linear2 = 3 [I, 0]: 3 silu(y)
      linear_out = 0 and pointwise_conv2 = 0: the attention and conv branches add 0
      r1 = x + 0.5 silu(LN(x));  r4 = r1 + 0.5 * 3 silu(LN(r1));  out = LN(r4)
    For x = [1, -1, 2, -2]: LN(x) = x / sqrt(2.5 + 1e-5) = [0.63245, -0.63245,
    1.26491, -1.26491]; silu = [0.41302, -0.21943, 0.98646, -0.27846];
    r1 = [1.20651, -1.10972, 2.49323, -2.13922] (mean 0.11270, variance
    3.35721); LN(r1) = [0.59697, -0.66716, 1.29923, -1.22904]; 3 silu =
    [1.15507, -0.67875, 3.06245, -0.83456]; r4 = [1.78405, -1.44910, 4.02444,
    -2.55651] (mean 0.45073, variance 6.80051); out = [0.51129, -0.72852,
    1.37041, -1.15318].  The second frame [0.5, 0.25, -1, 3] the same way."""
    enc = _encoder(D=4, H=2, Ly=1, left=2, right=1, K=3, bias=False, seed=11)
    layer = enc.layers[0]
    eye = torch.eye(4, dtype=torch.float64)
    with torch.no_grad():
        for mod in layer.modules():
            if isinstance(mod, torch.nn.LayerNorm):
                mod.weight.fill_(1.0)
                mod.bias.zero_()
        for ff, scale in ((layer.feed_forward1, 1.0), (layer.feed_forward2, 3.0)):
            ff.linear1.weight.zero_()
            ff.linear1.weight[:4] = eye
            ff.linear2.weight.zero_()
            ff.linear2.weight[:, :4] = scale * eye
        layer.self_attn.linear_out.weight.zero_()
        layer.conv.pointwise_conv2.weight.zero_()
    st = oe.EncoderState(1, 1, 2, 1, 4, 3)
    x = np.array([[[1.0, -1.0, 2.0, -2.0], [0.5, 0.25, -1.0, 3.0]]])
    got = oe.encoder_step(x, _state_dict(enc), st, np.full(1, 2), 1, 2, relpos.sinusoid_table(64, 4).astype(np.float64))
    want = np.array([[0.51129, -0.72852, 1.37041, -1.15318], [-0.28181, -0.41795, -0.97319, 1.67296]])
    np.testing.assert_allclose(got[0].T, want, atol=2e-5)
