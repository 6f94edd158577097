"""The drop-in encoder's own module tree run on the CPU in float64 with the
paged parts replaced by the oracle, for the composed parity tests:

* every layer's ConformerAttention.forward -> the module's projections, the
  dense shift-buffer update (cache.py:36-45) and the oracle's rel-pos attention
  (attention.py:85-125);
* every layer's ConformerConvolution.forward -> the module's pointwise
  projections around the oracle's streaming step over the dense [B, D, K-1]
  conv cache (convolution.py:150-162, cache.py:47-53);
* _create_streaming_masks -> the oracle's per-stream loop (encoder.py:167-227).

The layer composition (encoder.py:50-81), the feed-forward blocks and the
LayerNorms stay the module's; ``oracle/encoder.py`` restates those too, and
test_oracle_encoder.py checks the two against each other.
"""

from __future__ import annotations

import copy
import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle import attention as oa
from oracle import conv as oc
from oracle import masks as om


def dense_shift(win, slot, layer, left, new):
    """cache.py:37-44 for one stream: keep the last `left` frames, append."""
    if left > 0:
        win[slot, layer, :left] = win[slot, layer, -left:].copy()
    win[slot, layer, left:] = new


def init_attention(att, D, seed):
    """Projections ~ N(0, 1/D), rel-pos biases ~ N(0, 0.02^2)."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for lin in (att.qkv, att.linear_pos, att.linear_out):
            lin.weight.copy_(torch.randn(lin.weight.shape, generator=g) / math.sqrt(D))
        att.pos_bias_u.copy_(torch.randn(att.pos_bias_u.shape, generator=g) * 0.02)
        att.pos_bias_v.copy_(torch.randn(att.pos_bias_v.shape, generator=g) * 0.02)


class DenseCache:
    """Dense per-stream cache for the CPU reference encoder: K/V shift buffers
    (cache.py:19-45) and the conv cache (cache.py:30-34,47-53)."""

    def __init__(self, B, Ly, left, right, D, K):
        self.left = left
        self.k = np.zeros((B, Ly, left + right + 1, D))
        self.v = np.zeros_like(self.k)
        self.conv = torch.zeros(B, Ly, D, K - 1, dtype=torch.float64)

    def get_conv_cache(self, layer):
        return self.conv[:, layer]

    def update_conv_cache(self, layer, state):
        self.conv[:, layer] = state

    conv_ref = get_conv_cache  # the CPU reference's conv step takes the state tensor


def oracle_conv(conv):
    """Replaces ConformerConvolution.forward on the CPU reference."""

    def forward(x, pad_mask, cache=None):
        bn, dw = conv.batch_norm, conv.depthwise_conv
        h = F.linear(x, conv.pointwise_conv1.weight.squeeze(-1), conv.pointwise_conv1.bias).numpy()
        dw_bias = None if dw.bias is None else dw.bias.detach().numpy()
        y, nxt = oc.conv_module_step(
            h, cache.transpose(1, 2).numpy(), pad_mask.numpy(), dw.weight.detach().numpy().reshape(conv.d_model, -1),
            dw_bias, bn.weight.detach().numpy(), bn.bias.detach().numpy(), bn.eps,
        )
        out = F.linear(torch.from_numpy(y), conv.pointwise_conv2.weight.squeeze(-1), conv.pointwise_conv2.bias)
        return out, torch.from_numpy(nxt).transpose(1, 2)

    return forward


def torch_residual_norm(residual, branch, norm, alpha, in_place=False):
    """encoder.py:61-80 as torch ops: ``residual += x * 0.5`` (or ``+= x``), then
    the LayerNorm that reads it; replaces the layer's one-launch form on the CPU
    reference."""
    residual = residual + (branch * alpha if alpha != 1.0 else branch)
    return residual, norm(residual)


def oracle_attention(att, left, H):
    """Replaces ConformerAttention.forward on the CPU reference."""

    def forward(x, pos_emb, attn_mask=None, cache=None):
        q, k, v = (t.numpy() for t in att.qkv(x).chunk(3, dim=-1))
        pos = att.linear_pos(pos_emb)[0].numpy()
        layer = att.layer_idx
        for b in range(x.shape[0]):
            dense_shift(cache.k, b, layer, left, k[b])
            dense_shift(cache.v, b, layer, left, v[b])
        core = oa.relpos_attention(
            q, cache.k[:, layer], cache.v[:, layer], pos,
            att.pos_bias_u.detach().numpy(), att.pos_bias_v.detach().numpy(), attn_mask.numpy(), H,
        )
        return att.linear_out(torch.from_numpy(core))

    return forward


def module_reference(enc, H):
    """A float64 CPU copy of ``enc`` with attention, conv steps and masks from
    the oracle; step it with ``ref(x, StreamingState(DenseCache, proc, cl), length)``."""
    left, right = enc.att_context_size
    ref = copy.deepcopy(enc).double().cpu()
    for layer in ref.layers:
        layer.self_attn.forward = oracle_attention(layer.self_attn, left, H)
        layer.conv.forward = oracle_conv(layer.conv)
        layer.residual_norm = torch_residual_norm

    def ref_masks(current_len, cache_lengths, processed_frames, device, lengths):
        pad, att = om.create_streaming_masks(
            current_len, cache_lengths.numpy(), processed_frames.numpy(), lengths.numpy(), (left, right)
        )
        return torch.from_numpy(pad), torch.from_numpy(att)

    ref._create_streaming_masks = ref_masks
    return ref
