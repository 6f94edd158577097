"""CPU checks of the drop-in modules' boundary:

* ``PositionalEncoding`` (parakeet/modules/attention.py:23-62): the table
  ``extend_pe`` builds against the committed golden table
  (tests/golden/sinusoid.npz, written by tests/golden/make_golden.py) and the
  ``forward`` slice against the closed form sin / cos of the relative
  positions it stands for, evaluated in float64 with ``math``;
* ``ConformerEncoder``'s parameter names and shapes against the reference's
  module tree, enumerated here from the reference's constructors
  (encoder.py:11-48,84-138, subsample.py:60-139, attention.py:65-77,
  convolution.py:107-148, feedforward.py:4-18), and a strict
  ``load_state_dict`` of a state dict built from that enumeration (what
  ``Parakeet.from_pretrained`` does, model.py:126).
"""

import math
import os

import numpy as np
import pytest
import torch

from parakeet_amd.modules.attention import PositionalEncoding
from parakeet_amd.modules.encoder import ConformerEncoder
from parakeet_amd.modules.frontend import ConvSubsampling

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("length,d_model", [(9, 16), (143, 32)])
def test_positional_encoding_table_matches_golden(length, d_model):
    g = np.load(os.path.join(GOLDEN, "sinusoid.npz"))[f"len{length}_d{d_model}"]
    pe = PositionalEncoding(hidden_size=d_model, dropout=0.0, max_len=length, dropout_rate_emb=0.0)
    pe.extend_pe(length, device="cpu")
    got = pe.pe[0].numpy()
    assert got.shape == g.shape == (2 * length - 1, d_model)
    # same float32 torch arithmetic as the golden writer; the bound is the one
    # the oracle's table meets (an ulp of a frequency times |pos|)
    np.testing.assert_allclose(got, g, rtol=0, atol=length * 2.0**-23 + 2.0**-23)


@pytest.mark.parametrize("T,left", [(2, 70), (14, 70), (3, 5)])
def test_positional_encoding_forward_slice_is_relative_positions(T, left):
    d_model, max_len = 64, 5000
    pe = PositionalEncoding(hidden_size=d_model, dropout=0.0, max_len=max_len, dropout_rate_emb=0.0)
    pe.extend_pe(max_len, device="cpu")
    x = torch.randn(2, T, d_model)
    x_out, pos_emb = pe(x, cache_len=left)
    assert torch.equal(x_out, x)
    L = T + left
    assert tuple(pos_emb.shape) == (1, 2 * L - 1, d_model)
    # row r stands for relative position (L - 1) - r (attention.py:55-62):
    # even columns sin(pos * w_k), odd columns cos(pos * w_k),
    # w_k = exp(-2k ln(10000) / d_model)
    rel = (L - 1) - np.arange(2 * L - 1, dtype=np.float64)
    w = np.array([math.exp(-(2 * k) * math.log(10000.0) / d_model) for k in range(d_model // 2)])
    ang = rel[:, None] * w[None, :]
    ref = np.empty((2 * L - 1, d_model))
    ref[:, 0::2] = np.sin(ang)
    ref[:, 1::2] = np.cos(ang)
    # float32 angle rounding: |pos * w| <= L, an ulp of the product and of w
    np.testing.assert_allclose(pos_emb[0].double().numpy(), ref, rtol=0, atol=4 * L * 2.0**-23 + 2.0**-22)


def _freq_dim(feat_in, repeat=3, k=3, s=2, pad=3):
    # subsample.py:9-15 calc_length with all_paddings = (k - 1) + (s - 1)
    n = feat_in
    for _ in range(repeat):
        n = math.floor((n + pad - k) / s + 1)
    return n


def reference_encoder_params(feat_in, hidden, ff_exp, layers, heads, conv_k, sub_ch, use_bias):
    """Parameter name -> shape of parakeet.modules.encoder.ConformerEncoder,
    enumerated from the reference's constructors (PositionalEncoding's ``pe``
    is a non-persistent buffer, attention.py:47, so it has no key)."""
    C, D, dk = sub_ch, hidden, hidden // heads
    p = {}
    # pre_encode: ConvSubsampling (encoder.py:105-112, subsample.py:81-139):
    # conv.0 CausalConv2D(1 -> C), conv.1 ReLU, then twice [depthwise C, pointwise C, ReLU]
    p["pre_encode.conv.0.weight"] = (C, 1, 3, 3)
    p["pre_encode.conv.0.bias"] = (C,)
    for dw, pw in ((2, 3), (5, 6)):
        p[f"pre_encode.conv.{dw}.weight"] = (C, 1, 3, 3)
        p[f"pre_encode.conv.{dw}.bias"] = (C,)
        p[f"pre_encode.conv.{pw}.weight"] = (C, C, 1, 1)
        p[f"pre_encode.conv.{pw}.bias"] = (C,)
    p["pre_encode.out.weight"] = (D, C * _freq_dim(feat_in))
    p["pre_encode.out.bias"] = (D,)
    for i in range(layers):
        pre = f"layers.{i}."
        for ln in ("norm_feed_forward1", "norm_conv", "norm_self_att", "norm_feed_forward2", "norm_out"):
            p[pre + ln + ".weight"] = (D,)
            p[pre + ln + ".bias"] = (D,)
        for ff in ("feed_forward1", "feed_forward2"):  # feedforward.py:4-18
            p[pre + ff + ".linear1.weight"] = (D * ff_exp, D)
            p[pre + ff + ".linear2.weight"] = (D, D * ff_exp)
            if use_bias:
                p[pre + ff + ".linear1.bias"] = (D * ff_exp,)
                p[pre + ff + ".linear2.bias"] = (D,)
        # ConformerConvolution built without use_bias (encoder.py:30-32 -> convolution.py:107-148)
        p[pre + "conv.pointwise_conv1.weight"] = (2 * D, D, 1)
        p[pre + "conv.depthwise_conv.weight"] = (D, 1, conv_k)
        p[pre + "conv.batch_norm.weight"] = (D,)
        p[pre + "conv.batch_norm.bias"] = (D,)
        p[pre + "conv.pointwise_conv2.weight"] = (D, D, 1)
        # ConformerAttention (attention.py:65-77)
        for lin, rows in (("linear_out", D), ("linear_pos", D), ("qkv", 3 * D)):
            p[pre + f"self_attn.{lin}.weight"] = (rows, D)
            if use_bias:
                p[pre + f"self_attn.{lin}.bias"] = (rows,)
        p[pre + "self_attn.pos_bias_u"] = (heads, dk)
        p[pre + "self_attn.pos_bias_v"] = (heads, dk)
    return p


ENC_CASES = [
    # feat_in, hidden, ff_exp, layers, heads, conv_k, sub_ch, use_bias
    (80, 64, 4, 2, 2, 9, 16, False),
    (128, 96, 2, 1, 4, 5, 8, True),
]


@pytest.mark.parametrize("case", ENC_CASES)
def test_encoder_parameters_match_reference_tree(case):
    feat_in, hidden, ff_exp, layers, heads, conv_k, sub_ch, use_bias = case
    enc = ConformerEncoder(
        feat_in=feat_in, hidden_size=hidden, ff_expansion_factor=ff_exp, num_layers=layers, num_heads=heads,
        subsampling_factor=8, pos_emb_max_len=64, conv_kernel_size=conv_k, att_context_size=(70, 1),
        subsampling_conv_channels=sub_ch, use_bias=use_bias,
    )
    got = {k: tuple(v.shape) for k, v in enc.state_dict().items()}
    want = reference_encoder_params(feat_in, hidden, ff_exp, layers, heads, conv_k, sub_ch, use_bias)
    assert set(got) == set(want), (sorted(set(got) - set(want)), sorted(set(want) - set(got)))
    assert got == want
    assert isinstance(enc.pre_encode, ConvSubsampling)


def test_encoder_loads_reference_shaped_state_dict_strictly():
    feat_in, hidden, ff_exp, layers, heads, conv_k, sub_ch, use_bias = ENC_CASES[0]
    enc = ConformerEncoder(
        feat_in=feat_in, hidden_size=hidden, ff_expansion_factor=ff_exp, num_layers=layers, num_heads=heads,
        subsampling_factor=8, pos_emb_max_len=64, conv_kernel_size=conv_k, att_context_size=(70, 1),
        subsampling_conv_channels=sub_ch, use_bias=use_bias,
    )
    g = torch.Generator().manual_seed(0)
    sd = {k: torch.randn(shape, generator=g) for k, shape in reference_encoder_params(*ENC_CASES[0]).items()}
    res = enc.load_state_dict(sd, strict=True)
    assert not res.missing_keys and not res.unexpected_keys
    for k, v in enc.state_dict().items():
        assert torch.equal(v, sd[k]), k


def test_stream_tokens_read_like_per_stream_lists():
    """The decode step's lazy per-stream result against the per-frame lists of
    the same step concatenated per stream, including streams whose length cuts
    frames off (their counts must not show) and empty streams."""
    import numpy as np

    from parakeet_amd.modules.decoder import GreedyDecoder, StreamTokens

    rng = np.random.default_rng(7)
    B, T, S = 37, 3, 5
    cnt = rng.integers(0, S + 1, size=(B, T)).astype(np.int32)
    tok = np.full((B, T * S), -1, dtype=np.int32)
    for b in range(B):
        n = int(cnt[b].sum())
        tok[b, :n] = rng.integers(0, 1000, size=n)
    lens = rng.integers(0, T + 1, size=B).astype(np.int32)
    per_frame = GreedyDecoder._split(tok, cnt, lens, True)
    want = [sum(frames, []) for frames in per_frame]
    got = GreedyDecoder._split(tok, cnt, lens, False)
    assert isinstance(got, StreamTokens) and len(got) == B
    assert got == want and [got[b] for b in range(B)] == want and got[-1] == want[-1] and got[2:5] == want[2:5]
    assert got.counts().tolist() == [len(w) for w in want] and got.total() == sum(map(len, want))
    assert got.flat().tolist() == sum(want, []) and got.offsets()[-1] == got.total()
    empty = GreedyDecoder._split(tok[:0], cnt[:0], lens[:0], False)
    assert len(empty) == 0 and empty == []
