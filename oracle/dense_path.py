"""The reference's dense encoder-attention step on the CPU (torch, fp32).

This is the timed CPU baseline: one step gathers the batch's dense state out of
the slot pool (parakeet/engine/scheduler.py:128-170), builds the streaming masks
with the per-stream loop (parakeet/modules/encoder.py:167-227), runs every
layer's cache shift (parakeet/modules/cache.py:36-45) and rel-pos attention
(parakeet/modules/attention.py:94-121 via ``relpos_attention_torch``), advances
the state scalars (encoder.py:257-260) and scatters the state back
(scheduler.py:172-201).  The qkv / linear_pos / linear_out projections are
outside the hot path on both sides and are not run.  fp32 is the only dtype the
reference runs (its -1e5 mask overflows fp16).  Test infrastructure only.
"""

from __future__ import annotations

import torch

from .attention import relpos_attention_torch


def streaming_masks_torch(current_len, cache_lengths, processed_frames, lengths, att_context_size):
    """encoder.py:167-227 with the reference's torch ops and .item() reads."""
    chunk_size = att_context_size[1] + 1
    max_cache_len = att_context_size[0]
    left_chunks_num = att_context_size[0] // chunk_size
    batch = cache_lengths.shape[0]
    key_len_max = max_cache_len + current_len
    pad_mask = torch.zeros(batch, current_len, dtype=torch.bool)
    att_mask = torch.ones(batch, current_len, key_len_max, dtype=torch.bool)
    for idx in range(batch):
        cache_len = int(cache_lengths[idx].item())
        proc = int(processed_frames[idx].item())
        key_start = max(proc - cache_len, 0)
        key_len = cache_len + current_len
        key_pos = torch.arange(key_start, key_start + key_len, dtype=torch.int)
        query_pos = key_pos[-current_len:]
        chunk_idx_k = torch.div(key_pos, chunk_size, rounding_mode="trunc")
        chunk_idx_q = torch.div(query_pos, chunk_size, rounding_mode="trunc")
        diff_chunks = chunk_idx_q.unsqueeze(1) - chunk_idx_k.unsqueeze(0)
        allowed = torch.logical_and(torch.le(diff_chunks, left_chunks_num), torch.ge(diff_chunks, 0))
        valid_current = torch.arange(current_len) < lengths[idx]
        pad_mask[idx] = ~valid_current
        valid_total = torch.zeros(cache_len + current_len, dtype=torch.bool)
        if cache_len:
            valid_total[:cache_len] = True
        valid_total[cache_len : cache_len + current_len] = valid_current
        offset = max_cache_len - cache_len
        allowed_full = torch.zeros(current_len, key_len_max, dtype=torch.bool)
        allowed_full[:, offset : offset + key_len] = allowed
        valid_total_full = torch.zeros(key_len_max, dtype=torch.bool)
        valid_total_full[offset : offset + key_len] = valid_total
        valid_for_att = valid_current.unsqueeze(1) & valid_total_full.unsqueeze(0)
        att_mask[idx] = ~torch.logical_and(allowed_full, valid_for_att)
    return pad_mask, att_mask


class DenseStatePool:
    """Slot pool of dense state: attn_k/attn_v [N, Ly, L, D], conv [N, Ly, D, K-1],
    processed_frames / cache_lengths [N] (cache.py:24-34, encoder.py:159-160)."""

    def __init__(self, num_slots, num_layers, left, right, d_model, conv_kernel=9, dtype=torch.float32):
        self.left, self.right = left, right
        self.L = left + right + 1
        self.attn_k = torch.zeros(num_slots, num_layers, self.L, d_model, dtype=dtype)
        self.attn_v = torch.zeros_like(self.attn_k)
        self.conv = torch.zeros(num_slots, num_layers, d_model, conv_kernel - 1, dtype=dtype)
        self.processed = torch.zeros(num_slots, dtype=torch.int64)
        self.cache_len = torch.zeros(num_slots, dtype=torch.int64)
        self._batch = None

    def reset_slot(self, s):
        """scheduler.py:86-91 + cache.py:60-63."""
        self.processed[s] = 0
        self.cache_len[s] = 0
        self.attn_k[s].zero_()
        self.attn_v[s].zero_()
        self.conv[s].zero_()

    def step(self, slots, qkv_layers, pos, bias_u, bias_v, num_heads):
        """One encoder-attention step for the streams in ``slots``.

        qkv_layers: per layer a [B, T, 3D] fp32 tensor (q | k | v);
        pos: [2L-1, D]; returns the last layer's attention output [B, T, D]."""
        idx = torch.as_tensor(slots, dtype=torch.long)
        B = idx.shape[0]
        Ly = self.attn_k.shape[1]
        # pack_states (scheduler.py:128-170): batch buffers, then 5 index_selects
        if self._batch is None or self._batch[0].shape[0] < B:
            self._batch = (
                torch.empty((B,) + tuple(self.attn_k.shape[1:]), dtype=self.attn_k.dtype),
                torch.empty((B,) + tuple(self.attn_v.shape[1:]), dtype=self.attn_v.dtype),
                torch.empty((B,) + tuple(self.conv.shape[1:]), dtype=self.conv.dtype),
                torch.empty(B, dtype=torch.int64),
                torch.empty(B, dtype=torch.int64),
            )
        bk, bv, bc, bp, bl = (t[:B] for t in self._batch)
        torch.index_select(self.processed, 0, idx, out=bp)
        torch.index_select(self.cache_len, 0, idx, out=bl)
        torch.index_select(self.attn_k, 0, idx, out=bk)
        torch.index_select(self.attn_v, 0, idx, out=bv)
        torch.index_select(self.conv, 0, idx, out=bc)
        T = qkv_layers[0].shape[1]
        length = torch.full((B,), T, dtype=torch.int64)
        _, att_mask = streaming_masks_torch(T, bl, bp, length, (self.left, self.right))
        out = None
        for layer in range(Ly):
            q, k, v = qkv_layers[layer][:B].chunk(3, dim=-1)
            # update_attn_cache (cache.py:36-45)
            left = self.left
            bk[:, layer, :left].copy_(bk[:, layer, -left:].clone())
            bv[:, layer, :left].copy_(bv[:, layer, -left:].clone())
            bk[:, layer, left:].copy_(k)
            bv[:, layer, left:].copy_(v)
            out = relpos_attention_torch(q, bk[:, layer], bv[:, layer], pos, bias_u, bias_v, att_mask, num_heads)
        # encoder.py:257-260
        bp.add_(length)
        bl.add_(length)
        bl.clamp_(max=self.left)
        # unpack_states (scheduler.py:172-201)
        self.processed.index_copy_(0, idx, bp)
        self.cache_len.index_copy_(0, idx, bl)
        self.attn_k.index_copy_(0, idx, bk)
        self.attn_v.index_copy_(0, idx, bv)
        self.conv.index_copy_(0, idx, bc)
        return out
