"""ConformerAttention core of the reference, restated.

``relpos_attention`` follows parakeet/modules/attention.py:94-125 operation for
operation in numpy (float64 by default): bd = (q+v)·posᵀ, rel_shift, slice to
the key length, ×1/√dk, masked_fill(-1e5), then SDPA's softmax((q+u)·kᵀ/√dk +
bd)·V (attention.py:9-20).  ``relpos_attention_torch`` is the same sequence in
torch fp32 on the CPU with torch's own SDPA -- the reference's exact operator
path, used as the timed CPU baseline and to cross-check the numpy form.
Test infrastructure only.
"""

from __future__ import annotations

import math

import numpy as np

from .relpos import rel_shift


def relpos_attention(q, k, v, pos, bias_u, bias_v, mask, num_heads, dtype=np.float64):
    """q: [B, T, D]; k, v: [B, L, D] (the window); pos: [P, D] (linear_pos output,
    P >= L + T - 1); bias_u/v: [H, dk]; mask: [B, T, L] bool (True = masked) or
    None.  Returns [B, T, D] before linear_out."""
    q, k, v, pos = (np.asarray(a, dtype=dtype) for a in (q, k, v, pos))
    bias_u = np.asarray(bias_u, dtype=dtype)
    bias_v = np.asarray(bias_v, dtype=dtype)
    B, T, D = q.shape
    L = k.shape[1]
    H = num_heads
    dk = D // H
    qh = q.reshape(B, T, H, dk)  # :108 view
    kh = k.reshape(B, L, H, dk).transpose(0, 2, 1, 3)  # :109
    vh = v.reshape(B, L, H, dk).transpose(0, 2, 1, 3)  # :110
    ph = pos.reshape(1, -1, H, dk).transpose(0, 2, 1, 3)  # :102-106
    q_u = (qh + bias_u).transpose(0, 2, 1, 3)  # :108
    q_v = (qh + bias_v).transpose(0, 2, 1, 3)  # :109
    bd = q_v @ ph.transpose(0, 1, 3, 2)  # :111
    bd = rel_shift(bd)[:, :, :, :L] * (1.0 / math.sqrt(dk))  # :112-113
    if mask is not None:
        m = np.asarray(mask, dtype=bool)
        if m.ndim == 3:
            m = m[:, None]
        bd = np.where(m, dtype(-1e5), bd)  # :115
    scores = (q_u @ kh.transpose(0, 1, 3, 2)) * (1.0 / math.sqrt(dk)) + bd  # SDPA scale=None
    scores = scores - scores.max(axis=-1, keepdims=True)
    p = np.exp(scores)
    p = p / p.sum(axis=-1, keepdims=True)
    out = p @ vh  # [B, H, T, dk]
    return out.transpose(0, 2, 1, 3).reshape(B, T, D)  # :19, :122


def relpos_attention_direct(q, k, v, pos, bias_u, bias_v, mask, num_heads):
    """The same attention written per score with the relative row index
    r = j + T - 1 - i instead of the pad/view shift (float64 loops; tiny inputs)."""
    q, k, v, pos = (np.asarray(a, dtype=np.float64) for a in (q, k, v, pos))
    bias_u = np.asarray(bias_u, dtype=np.float64)
    bias_v = np.asarray(bias_v, dtype=np.float64)
    B, T, D = q.shape
    L = k.shape[1]
    H = num_heads
    dk = D // H
    out = np.zeros((B, T, D))
    for b in range(B):
        for h in range(H):
            sl = slice(h * dk, (h + 1) * dk)
            for i in range(T):
                s = np.empty(L)
                for j in range(L):
                    ac = float(np.dot(q[b, i, sl] + bias_u[h], k[b, j, sl]))
                    if mask is not None and mask[b, i, j]:
                        s[j] = ac / math.sqrt(dk) - 1e5
                    else:
                        bd = float(np.dot(q[b, i, sl] + bias_v[h], pos[j + T - 1 - i, sl]))
                        s[j] = (ac + bd) / math.sqrt(dk)
                w = np.exp(s - s.max())
                w /= w.sum()
                out[b, i, sl] = w @ v[b, :, sl]
    return out


def relpos_attention_torch(q, k, v, pos, bias_u, bias_v, mask, num_heads):
    """attention.py:94-123 (without the projections) with torch CPU ops in the
    input dtype: matmul, pad/view rel_shift, masked_fill(-1e5), SDPA."""
    import torch
    import torch.nn.functional as F

    B, T, D = q.shape
    L = k.shape[1]
    H = num_heads
    dk = D // H
    query = q.view(B, T, H, dk)
    key = k.view(B, L, H, dk).transpose(1, 2)
    value = v.view(B, L, H, dk).transpose(1, 2)
    p = pos.view(1, -1, H, dk).transpose(1, 2)
    q_u = (query + bias_u).transpose(1, 2)
    q_v = (query + bias_v).transpose(1, 2)
    bd = torch.matmul(q_v, p.transpose(-2, -1))
    Bq, Hq, qlen, plen = bd.shape
    bd = F.pad(bd, pad=(1, 0)).view(Bq, Hq, -1, qlen)[:, :, 1:].view(Bq, Hq, qlen, plen)
    bd = bd[:, :, :, :L] * (1 / math.sqrt(dk))
    if mask is not None:
        m = mask.bool()
        if m.ndim == 3:
            m = m.unsqueeze(1)
        bd = bd.masked_fill(m, -1e5)
    out = F.scaled_dot_product_attention(q_u, key, value, attn_mask=bd, dropout_p=0.0, scale=None)
    return out.transpose(1, 2).contiguous().reshape(B, T, D)
