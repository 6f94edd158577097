"""Streaming step of the reference's Conformer convolution module, restated.

Test infrastructure only.

``conv_module_step`` follows parakeet/modules/convolution.py:150-158 from the
GLU to the activation, together with CausalConv1d.update_cache
(convolution.py:37-47) and the cache read / write of ModelCache
(parakeet/modules/cache.py:47-53):

    g      = glu(pointwise_conv1(x))           convolution.py:152-153 (channel dim)
    g      = g masked to 0 on padded frames    :155
    x~     = cat(cache, g) along time          :43-44  (right padding 0 for a causal conv)
    cache' = x~[last kernel-1 frames]          :46
    y      = depthwise conv1d(x~)              :47, Conv1d(groups=d_model), no padding
    y      = silu(layer_norm(y))               :156-157 (``batch_norm`` is a LayerNorm)

Layouts here are frame-major: ``h`` is [B, T, 2*D] (the pointwise-conv1 output
with channels last) and the cache is [B, kernel-1, D] -- row r is column r of the
reference's [B, D, kernel-1] cache.  The two pointwise convolutions (kernel size
1) are plain matrix products outside this step.

``round_to`` rounds the GLU output to a storage dtype before it enters the
window, as the reference's cat of model-dtype tensors holds it.
"""

from __future__ import annotations

import numpy as np
import torch


def round_to(x: np.ndarray, dtype: torch.dtype | None) -> np.ndarray:
    """x rounded to ``dtype`` (round to nearest even) and back to float64."""
    if dtype is None or dtype == torch.float64:
        return np.asarray(x, dtype=np.float64)
    return torch.from_numpy(np.asarray(x, dtype=np.float64)).to(dtype).double().numpy()


def glu(h: np.ndarray) -> np.ndarray:
    """F.glu over the channel dim (convolution.py:153): first half * sigmoid(second)."""
    h = np.asarray(h, dtype=np.float64)
    D = h.shape[-1] // 2
    return h[..., :D] / (1.0 + np.exp(-h[..., D:]))


def conv_module_step(h, cache, pad_mask, dw_weight, dw_bias, ln_weight, ln_bias, eps=1e-5, store_dtype=None):
    """One streaming step for B streams.

    h: [B, T, 2D]; cache: [B, K-1, D]; pad_mask: [B, T] bool (True = padded) or
    None; dw_weight: [D, K] (Conv1d weight [D, 1, K]); dw_bias: [D] or None;
    ln_weight, ln_bias: [D].  Returns (y [B, T, D], next cache [B, K-1, D]), both
    float64; the next cache holds frames already rounded to ``store_dtype``."""
    h = np.asarray(h, dtype=np.float64)
    cache = np.asarray(cache, dtype=np.float64)
    w = np.asarray(dw_weight, dtype=np.float64)
    B, T, _ = h.shape
    D, K = w.shape
    g = round_to(glu(h), store_dtype)  # [B, T, D]
    if pad_mask is not None:
        g = np.where(np.asarray(pad_mask, dtype=bool)[:, :, None], 0.0, g)
    x = np.concatenate([cache, g], axis=1)  # [B, K-1+T, D]
    nxt = x[:, x.shape[1] - (K - 1) :].copy()
    y = np.zeros((B, T, D))
    for k in range(K):  # Conv1d is a cross-correlation: out[t] = sum_k w[k] x[t+k]
        y += x[:, k : k + T, :] * w[:, k]
    if dw_bias is not None:
        y += np.asarray(dw_bias, dtype=np.float64)
    mean = y.mean(axis=-1, keepdims=True)
    var = ((y - mean) ** 2).mean(axis=-1, keepdims=True)
    z = (y - mean) / np.sqrt(var + eps) * np.asarray(ln_weight, dtype=np.float64) + np.asarray(ln_bias, dtype=np.float64)
    return z / (1.0 + np.exp(-z)), nxt


def conv_module_step_torch(h, cache_cm, pad_mask, dw_weight, dw_bias, ln_weight, ln_bias, eps=1e-5):
    """The same step as the reference writes it, operator for operator, in torch
    (convolution.py:150-158 with CausalConv1d.forward :49-52): channel-major
    tensors, F.glu(dim=1), masked_fill, torch.cat with the [B, D, K-1] cache,
    F.conv1d(groups=D), LayerNorm over the channels after a transpose, SiLU.
    h: [B, T, 2D] torch; cache_cm: [B, D, K-1] torch.  Returns (y [B, T, D],
    next cache [B, D, K-1])."""
    import torch.nn.functional as F

    x = h.transpose(1, 2)  # the pointwise-conv1 output in the reference's [B, 2D, T]
    x = F.glu(x, dim=1)
    if pad_mask is not None:
        x = x.masked_fill(pad_mask.unsqueeze(1), 0.0)
    new_x = torch.cat([cache_cm, F.pad(x, pad=(0, 0))], dim=-1)
    next_cache = new_x[:, :, -cache_cm.size(-1) :]
    D = new_x.shape[1]
    y = F.conv1d(new_x, dw_weight.reshape(D, 1, -1), dw_bias, groups=D)
    y = F.layer_norm(y.transpose(1, 2), (D,), ln_weight, ln_bias, eps)
    return F.silu(y), next_cache
