"""Dense shift-buffer cache of the reference, restated in numpy.

Follows parakeet/modules/cache.py:7-77 and the slot reset of
parakeet/engine/scheduler.py:86-91.  Test infrastructure only.
"""

from __future__ import annotations

import numpy as np


class DenseCache:
    """attn_k / attn_v: [N, Ly, left+right+1, D], zero-initialised (cache.py:19-29)."""

    def __init__(self, num_layers: int, left: int, right: int, d_model: int, batch: int, dtype=np.float32):
        self.left = int(left)
        self.right = int(right)
        self.L = self.left + self.right + 1  # cache.py:22
        self.attn_k = np.zeros((batch, num_layers, self.L, d_model), dtype=dtype)
        self.attn_v = np.zeros_like(self.attn_k)

    def update_attn_cache(self, layer: int, key: np.ndarray, value: np.ndarray):
        """cache.py:36-45: shift the last `left` frames to the front, write the
        new right+1 frames at the tail, return the layer's window."""
        left = self.left
        for buf, new in ((self.attn_k, key), (self.attn_v, value)):
            tail = buf[:, layer, -left:].copy() if left > 0 else None  # .clone() (cache.py:38)
            if left > 0:
                buf[:, layer, :left] = tail
            buf[:, layer, left:] = new
        return self.attn_k[:, layer], self.attn_v[:, layer]

    def reset_slot(self, slot: int) -> None:
        """cache.py:60-63."""
        self.attn_k[slot] = 0
        self.attn_v[slot] = 0


def window_closed_form(history: np.ndarray, appended: int, L: int) -> np.ndarray:
    """What the dense window must hold, stated from positions alone: after
    `appended` frames the window row j is frame appended - L + j, or zeros when
    that position is negative.  history: [appended, D] frames in append order."""
    D = history.shape[1]
    out = np.zeros((L, D), dtype=history.dtype)
    for j in range(L):
        p = appended - L + j
        if p >= 0:
            out[j] = history[p]
    return out
