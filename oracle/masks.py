"""Streaming masks of the reference, restated in numpy.

``create_streaming_masks`` follows ConformerEncoder._create_streaming_masks
(parakeet/modules/encoder.py:167-227) loop for loop.  ``masks_by_position`` is an
independent statement of the same rule in absolute frame positions, used to pin
the loop form.  True = masked (att_mask) / padded (pad_mask).  Test
infrastructure only.
"""

from __future__ import annotations

import numpy as np


def create_streaming_masks(current_len, cache_lengths, processed_frames, lengths, att_context_size):
    """encoder.py:167-227."""
    chunk_size = att_context_size[1] + 1  # :175
    max_cache_len = att_context_size[0]  # :176
    left_chunks_num = att_context_size[0] // chunk_size  # :177
    batch = len(cache_lengths)
    key_len_max = max_cache_len + current_len  # :180
    pad_mask = np.zeros((batch, current_len), dtype=bool)
    att_mask = np.ones((batch, current_len, key_len_max), dtype=bool)
    lengths = np.broadcast_to(np.asarray(lengths, dtype=np.int64), (batch,))
    for idx in range(batch):
        cache_len = int(cache_lengths[idx])  # :187
        proc = int(processed_frames[idx])  # :188
        key_start = max(proc - cache_len, 0)  # :189
        key_len = cache_len + current_len  # :190
        key_pos = np.arange(key_start, key_start + key_len, dtype=np.int64)  # :191-193
        query_pos = key_pos[-current_len:]  # :194
        chunk_idx_k = key_pos // chunk_size  # :196 (non-negative: trunc == floor)
        chunk_idx_q = query_pos // chunk_size  # :197
        diff_chunks = chunk_idx_q[:, None] - chunk_idx_k[None, :]  # :199
        allowed = (diff_chunks <= left_chunks_num) & (diff_chunks >= 0)  # :200-202
        valid_current = np.arange(current_len) < lengths[idx]  # :204
        pad_mask[idx] = ~valid_current  # :205
        valid_total = np.zeros(cache_len + current_len, dtype=bool)  # :207-209
        if cache_len:
            valid_total[:cache_len] = True
        valid_total[cache_len : cache_len + current_len] = valid_current  # :212
        offset = max_cache_len - cache_len  # :214
        allowed_full = np.zeros((current_len, key_len_max), dtype=bool)
        allowed_full[:, offset : offset + key_len] = allowed  # :218
        valid_total_full = np.zeros(key_len_max, dtype=bool)
        valid_total_full[offset : offset + key_len] = valid_total  # :221
        valid_for_att = valid_current[:, None] & valid_total_full[None, :]  # :223
        att_mask[idx] = ~(allowed_full & valid_for_att)  # :224-225
    return pad_mask, att_mask


def masks_by_position(current_len, cache_lengths, processed_frames, lengths, att_context_size):
    """Same rule stated per dense column: column j holds absolute frame
    kp = proc - left + j (proc >= cache_len); it is attendable by query i (frame
    proc + i) iff the key is one of the cache_len cached frames or a valid frame
    of this chunk, the query is valid, and the key's chunk is between the
    query's chunk - left//chunk_size and the query's chunk."""
    left, right = att_context_size
    C = right + 1
    batch = len(cache_lengths)
    lengths = np.broadcast_to(np.asarray(lengths, dtype=np.int64), (batch,))
    att = np.ones((batch, current_len, left + current_len), dtype=bool)
    pad = np.zeros((batch, current_len), dtype=bool)
    for b in range(batch):
        cl, proc, n = int(cache_lengths[b]), int(processed_frames[b]), int(lengths[b])
        assert proc >= cl, "streaming state keeps cache_len <= processed frames"
        for i in range(current_len):
            pad[b, i] = i >= n
            qp = proc + i
            for j in range(left + current_len):
                kp = proc - left + j
                cached = proc - cl <= kp < proc
                current = proc <= kp < proc + n
                chunk_ok = qp // C - left // C <= kp // C <= qp // C if kp >= 0 else False
                att[b, i, j] = not ((cached or current) and i < n and chunk_ok)
    return pad, att
