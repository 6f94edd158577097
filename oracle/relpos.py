"""Relative-position table and Transformer-XL shift of the reference, restated.

Test infrastructure only.
"""

from __future__ import annotations

import math

import numpy as np


def sinusoid_table(length: int, d_model: int, dtype=np.float32) -> np.ndarray:
    """PositionalEncoding.extend_pe/create_pe (parakeet/modules/attention.py:33-49):
    rows for positions length-1 ... -(length-1); even columns sin(pos*w), odd
    columns cos(pos*w), w_k = exp(2k * -(ln 10000 / d_model)) computed in fp32."""
    positions = np.arange(length - 1, -length, -1, dtype=np.float32)[:, None]  # :45-47
    div_term = np.exp(np.arange(0, d_model, 2, dtype=np.float32) * np.float32(-(math.log(10000.0) / d_model)))  # :36-43
    angles = (positions * div_term).astype(np.float32)
    pe = np.zeros((positions.shape[0], d_model), dtype=np.float64)
    pe[:, 0::2] = np.sin(angles.astype(np.float64))
    pe[:, 1::2] = np.cos(angles.astype(np.float64))
    return pe.astype(dtype)


def pos_slice(pe: np.ndarray, current_len: int, cache_len: int) -> np.ndarray:
    """PositionalEncoding.forward (attention.py:55-62): the 2*(T+cache_len)-1 rows
    centred on relative position 0."""
    input_len = current_len + cache_len
    center = pe.shape[0] // 2 + 1
    return pe[center - input_len : center + input_len - 1]


def rel_shift(x: np.ndarray) -> np.ndarray:
    """ConformerAttention.rel_shift (attention.py:79-83): left-pad one zero
    column, view [.., pos_len+1, qlen], drop the first row, view back."""
    B, H, qlen, pos_len = x.shape
    padded = np.concatenate([np.zeros((B, H, qlen, 1), dtype=x.dtype), x], axis=-1)
    return padded.reshape(B, H, -1, qlen)[:, :, 1:].reshape(B, H, qlen, pos_len)
