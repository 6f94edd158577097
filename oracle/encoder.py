"""Streaming FastConformer encoder step of the reference, restated in float64.

Test infrastructure only.

One call of ``ConformerEncoder.forward`` (parakeet/modules/encoder.py:229-267)
on whole chunks, composed from the oracle's parts over dense per-stream caches:

* position table: ``relpos.sinusoid_table`` / ``relpos.pos_slice``
  (attention.py:33-62), sliced at ``cache_len = left`` (encoder.py:239);
* masks: ``masks.create_streaming_masks`` (encoder.py:167-227);
* per layer, ConformerLayer.forward (encoder.py:50-81):
      r  = x + 0.5 * FF1(LN_ff1(x))                       :58-61
      r += MHA(LN_att(r), pos, att_mask, cache)           :63-68
      r += Conv(LN_conv(r), pad_mask, conv cache)         :70-74
      r += 0.5 * FF2(LN_ff2(r))                           :76-78
      out = LN_out(r)                                     :80
  with FF = linear2(silu(linear1(.))) (feedforward.py:21-26), MHA = qkv
  projection, the dense shift-buffer update (cache.py:36-45),
  ``attention.relpos_attention`` and linear_out (attention.py:85-125), Conv =
  pointwise_conv1, ``conv.conv_module_step`` and pointwise_conv2
  (convolution.py:150-162, cache.py:47-53);
* state advance: processed += length, cache_len = min(cache_len + length, left)
  (encoder.py:257-260).

Weights come from a state dict whose keys are the reference module tree's
(``layers.{i}.self_attn.qkv.weight`` ...), as float64 numpy arrays.
"""

from __future__ import annotations

import numpy as np

from . import attention as oa
from . import conv as oc
from . import masks as om
from . import relpos


def layer_norm(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """nn.LayerNorm over the last dim (biased variance)."""
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def linear(x: np.ndarray, sd: dict, name: str) -> np.ndarray:
    y = x @ sd[name + ".weight"].T
    bias = sd.get(name + ".bias")
    return y if bias is None else y + bias


def silu(x: np.ndarray) -> np.ndarray:
    return x / (1.0 + np.exp(-x))


def feed_forward(x: np.ndarray, sd: dict, prefix: str) -> np.ndarray:
    """ConformerFeedForward.forward (feedforward.py:21-26), dropout off."""
    return linear(silu(linear(x, sd, prefix + ".linear1")), sd, prefix + ".linear2")


class EncoderState:
    """Dense per-stream caches of one batch: the K/V shift buffers
    [B, Ly, left+T, D] (cache.py:19-29), the conv cache [B, Ly, K-1, D]
    (frame-major: row r is column r of cache.py:30-34's [D, K-1]) and the
    processed_frames / cache_lengths counters (cache.py:80-89)."""

    def __init__(self, B: int, layers: int, left: int, right: int, d_model: int, kernel: int):
        self.left, self.right = left, right
        L = left + right + 1
        self.k = np.zeros((B, layers, L, d_model))
        self.v = np.zeros_like(self.k)
        self.conv = np.zeros((B, layers, kernel - 1, d_model))
        self.processed = np.zeros(B, dtype=np.int64)
        self.cache_len = np.zeros(B, dtype=np.int64)

    def reset_slot(self, b: int) -> None:
        self.k[b] = 0.0
        self.v[b] = 0.0
        self.conv[b] = 0.0
        self.processed[b] = 0
        self.cache_len[b] = 0


def _shift_append(win: np.ndarray, left: int, new: np.ndarray) -> None:
    """cache.py:37-44 on one layer's [B, L, D]: keep the last ``left`` frames, append."""
    if left > 0:
        win[:, :left] = win[:, -left:].copy()
    win[:, left:] = new


def attention(x, sd, prefix, layer, st: EncoderState, pos_emb, att_mask, heads):
    """ConformerAttention.forward (attention.py:85-125) with a dense cache."""
    qkv = linear(x, sd, prefix + ".qkv")
    q, k, v = np.split(qkv, 3, axis=-1)
    _shift_append(st.k[:, layer], st.left, k)
    _shift_append(st.v[:, layer], st.left, v)
    pos = linear(pos_emb, sd, prefix + ".linear_pos")
    core = oa.relpos_attention(
        q, st.k[:, layer], st.v[:, layer], pos, sd[prefix + ".pos_bias_u"], sd[prefix + ".pos_bias_v"], att_mask, heads
    )
    return linear(core, sd, prefix + ".linear_out")


def convolution(x, sd, prefix, layer, st: EncoderState, pad_mask):
    """ConformerConvolution.forward (convolution.py:150-162): pointwise_conv1
    (a [2D, D, 1] kernel), the oracle's GLU / masked causal depthwise step /
    LayerNorm / SiLU with the layer's conv cache, pointwise_conv2."""
    w1 = sd[prefix + ".pointwise_conv1.weight"][:, :, 0]
    h = x @ w1.T
    b1 = sd.get(prefix + ".pointwise_conv1.bias")
    if b1 is not None:
        h = h + b1
    dw = sd[prefix + ".depthwise_conv.weight"][:, 0, :]
    y, nxt = oc.conv_module_step(
        h, st.conv[:, layer], pad_mask, dw, sd.get(prefix + ".depthwise_conv.bias"),
        sd[prefix + ".batch_norm.weight"], sd[prefix + ".batch_norm.bias"],
    )
    st.conv[:, layer] = nxt
    w2 = sd[prefix + ".pointwise_conv2.weight"][:, :, 0]
    out = y @ w2.T
    b2 = sd.get(prefix + ".pointwise_conv2.bias")
    return out if b2 is None else out + b2


def conformer_layer(x, sd, layer, st: EncoderState, pos_emb, pad_mask, att_mask, heads):
    """ConformerLayer.forward (encoder.py:50-81)."""
    p = f"layers.{layer}"

    def ln(y, name):
        return layer_norm(y, sd[f"{p}.{name}.weight"], sd[f"{p}.{name}.bias"])

    r = x + 0.5 * feed_forward(ln(x, "norm_feed_forward1"), sd, p + ".feed_forward1")
    r = r + attention(ln(r, "norm_self_att"), sd, p + ".self_attn", layer, st, pos_emb, att_mask, heads)
    r = r + convolution(ln(r, "norm_conv"), sd, p + ".conv", layer, st, pad_mask)
    r = r + 0.5 * feed_forward(ln(r, "norm_feed_forward2"), sd, p + ".feed_forward2")
    return ln(r, "norm_out")


def encoder_step(x: np.ndarray, sd: dict, st: EncoderState, length: np.ndarray, layers: int, heads: int,
                 pe: np.ndarray) -> np.ndarray:
    """ConformerEncoder.forward (encoder.py:229-267) for x [B, T, D] (already
    subsampled, bypass_pre_encode) and per-stream ``length``; ``pe`` is the
    sinusoid table (``relpos.sinusoid_table(max_len, D)``).  Returns [B, D, T]
    and advances ``st``."""
    x = np.asarray(x, dtype=np.float64)
    T = x.shape[1]
    pos_emb = relpos.pos_slice(pe, T, st.left).astype(np.float64)
    pad_mask, att_mask = om.create_streaming_masks(T, st.cache_len, st.processed, length, (st.left, st.right))
    for layer in range(layers):
        x = conformer_layer(x, sd, layer, st, pos_emb, pad_mask, att_mask, heads)
    st.processed = st.processed + length
    st.cache_len = np.minimum(st.cache_len + length, st.left)
    return x.transpose(0, 2, 1)
