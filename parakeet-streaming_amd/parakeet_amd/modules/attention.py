"""Drop-in for ``parakeet.modules.attention`` (parakeet/modules/attention.py).

``ConformerAttention`` keeps the reference parameters (``qkv`` with rows in
[q; k; v] order, ``linear_pos``, ``linear_out``, ``pos_bias_u``, ``pos_bias_v``)
and ``forward(x, pos_emb, attn_mask, cache)``.  The three projections stay torch
GEMMs; everything between them -- cache update, (q+u)k^T, (q+v)p^T with the
Transformer-XL shift, the -1e5 mask, softmax and the value sum -- is one HIP
kernel reading the window straight from the cache pages.
"""

from __future__ import annotations

import math

import torch
from torch import Tensor, nn

from .. import ops
from .cache import ModelCache


class PositionalEncoding(nn.Module):
    """Sinusoidal relative-position table (parakeet/modules/attention.py:23-62).

    ``pe`` row r holds position (length-1) - r for r in [0, 2*length-1):
    even columns sin(pos * w_k), odd columns cos(pos * w_k) with
    w_k = exp(-(2k) * ln(10000) / hidden_size).  ``forward(x, cache_len)``
    returns ``x`` and the 2*(T+cache_len)-1 rows centred on position 0.
    """

    def __init__(self, hidden_size: int, dropout: float, max_len: int, dropout_rate_emb: float):
        super().__init__()
        self.hidden_size = hidden_size
        self.dropout = nn.Dropout(dropout)
        self.max_len = max_len
        self.dropout_emb = nn.Dropout(dropout_rate_emb)

    def create_pe(self, positions: Tensor) -> None:
        freqs = torch.exp(
            torch.arange(0, self.hidden_size, 2, dtype=torch.float32, device=positions.device)
            * -(math.log(10000.0) / self.hidden_size)
        )
        angles = positions * freqs
        pe = torch.zeros(positions.size(0), self.hidden_size, device=positions.device)
        pe[:, 0::2] = torch.sin(angles)
        pe[:, 1::2] = torch.cos(angles)
        self.register_buffer("pe", pe.unsqueeze(0), persistent=False)

    def extend_pe(self, length: int, device) -> None:
        positions = torch.arange(length - 1, -length, -1, dtype=torch.float32, device=device).unsqueeze(1)
        self.create_pe(positions=positions)

    def forward(self, x: Tensor, cache_len: int = 0):
        span = x.size(1) + cache_len
        centre = self.pe.size(1) // 2 + 1
        pos_emb = self.pe[:, centre - span : centre + span - 1]
        return self.dropout(x), self.dropout_emb(pos_emb)


class ConformerAttention(nn.Module):
    """Relative-position MHA (parakeet/modules/attention.py:65-125) on the paged cache."""

    def __init__(self, layer_idx, num_heads, hidden_size: int, use_bias: bool = False):
        super().__init__()
        self.layer_idx = layer_idx
        self.d_k = hidden_size // num_heads
        self.s_d_k = math.sqrt(self.d_k)
        self.num_heads = num_heads
        self.linear_out = nn.Linear(hidden_size, hidden_size, bias=use_bias)
        self.linear_pos = nn.Linear(hidden_size, hidden_size, bias=use_bias)
        self.qkv = nn.Linear(hidden_size, hidden_size * 3, bias=use_bias)
        self.pos_bias_u = nn.Parameter(torch.empty(self.num_heads, self.d_k))
        self.pos_bias_v = nn.Parameter(torch.empty(self.num_heads, self.d_k))
        # linear_pos(pos_emb), kept between steps: a streaming step's table is the
        # same slice of the same buffer every step (attention.py:102 recomputes it)
        self._pos_val: Tensor | None = None
        self._pos_key = None
        self._pos_src: Tensor | None = None

    def _pos_version(self, pos_emb: Tensor):
        """What the kept projection depends on: the table (address, shape, dtype,
        in-place version) and linear_pos's weight and bias; None when a version
        is not tracked (inference tensors), which disables keeping it."""
        try:
            parts = [pos_emb.data_ptr(), tuple(pos_emb.shape), tuple(pos_emb.stride()), pos_emb.dtype, pos_emb._version]
            for t in (self.linear_pos.weight, self.linear_pos.bias):
                parts += [None, None] if t is None else [t.data_ptr(), t._version]
        except RuntimeError:
            return None
        return tuple(parts)

    def projected_pos(self, pos_emb: Tensor) -> Tensor:
        """linear_pos(pos_emb), recomputed only when the table or the weights
        changed (always with gradients enabled).  A recomputation of the same
        shape is written into the kept buffer, which a recorded step reads."""
        if torch.is_grad_enabled():
            return self.linear_pos(pos_emb)
        key = self._pos_version(pos_emb)
        if key is None:
            return self.linear_pos(pos_emb)
        if key != self._pos_key:
            new = self.linear_pos(pos_emb)
            v = self._pos_val
            if v is not None and v.shape == new.shape and v.dtype == new.dtype and v.device == new.device:
                v.copy_(new)
            else:
                self._pos_val = new
            self._pos_key, self._pos_src = key, pos_emb
        return self._pos_val

    def refresh_projected_pos(self) -> None:
        """Recomputes the kept projection in place if the table or the weights
        changed since it was taken (a recorded step replays with the kept buffer)."""
        if self._pos_src is not None and self._pos_version(self._pos_src) != self._pos_key:
            with torch.no_grad():
                self.projected_pos(self._pos_src)

    def forward(self, x: Tensor, pos_emb: Tensor, attn_mask: Tensor, cache: ModelCache = None):
        B, T = x.shape[:2]
        qkv = self.qkv(x)
        query, key, value = qkv.chunk(3, dim=-1)
        # [1, P, D] is one table for every stream; [B, P, D] gives each stream
        # its own (the reference broadcasts both, attention.py:102-106)
        pos = self.projected_pos(pos_emb)
        if pos.dim() == 3 and pos.shape[0] == 1:
            pos = pos[0]
        mask = attn_mask.bool() if attn_mask is not None else None
        bias_u = self.pos_bias_u.to(x.dtype).contiguous()
        bias_v = self.pos_bias_v.to(x.dtype).contiguous()
        if cache is not None:
            out = cache.attend(
                self.layer_idx, query, key, value, pos, bias_u, bias_v, mask, num_heads=self.num_heads
            )
        else:
            out = ops.paged_relpos_attn(
                query, key, value, pos, bias_u, bias_v, mask, num_heads=self.num_heads, left=0, pages=None, append=False
            )
        return self.linear_out(out.reshape(B, T, self.num_heads * self.d_k))


__all__ = ["ConformerAttention", "PositionalEncoding"]
