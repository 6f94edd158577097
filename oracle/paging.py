"""Page pool, ring block table and page append/gather, restated in Python/numpy.

The reference has no pages: its per-slot dense buffer shifts by right+1 frames
per layer call (parakeet/modules/cache.py:36-45) and its free slots live in a
FIFO deque (parakeet/engine/scheduler.py:84 `deque(range(pool_size))`, :97
`popleft`, :104 `append`).  The paged build keeps that deque discipline for
pages: allocation pops the front, a freed page is appended to the back, and a
page is freed once no position of the slot's window [A+chunk-window, A+chunk)
lies in it -- the page-granular form of the shift at cache.py:37-42.
Test infrastructure only.
"""

from __future__ import annotations

from collections import deque

import numpy as np


def max_pages(left: int, chunk: int, page_size: int) -> int:
    window = left + chunk
    return (window + page_size - 2) // page_size + 1


class PagePoolModel:
    """Pure-Python model of the host page pool, one FIFO queue of free pages."""

    def __init__(self, num_pages, num_slots, page_size, left, chunk, page_order=None):
        self.P = int(page_size)
        self.left = int(left)
        self.chunk = int(chunk)
        self.window = self.left + self.chunk
        self.M = max_pages(self.left, self.chunk, self.P)
        if num_pages < num_slots * self.M:
            raise ValueError("pool too small for its slots")
        order = list(range(num_pages)) if page_order is None else [int(x) for x in page_order]
        if sorted(order) != list(range(num_pages)):
            raise ValueError("page_order is not a permutation")
        self.free = deque(order)
        self.appended = [0] * num_slots
        self.lo = [0] * num_slots
        self.hi = [0] * num_slots
        self.ring = [[-1] * self.M for _ in range(num_slots)]

    def advance(self, slots) -> np.ndarray:
        slots = [int(s) for s in slots]
        if len(set(slots)) != len(slots):
            raise ValueError("slot twice in one step")
        rows = np.empty((len(slots), 1 + self.M), dtype=np.int32)
        for b, s in enumerate(slots):
            end = self.appended[s] + self.chunk
            start = end - self.window
            # evict pages whose frames all precede the window
            while self.lo[s] < self.hi[s] and (self.lo[s] + 1) * self.P <= start:
                e = self.lo[s] % self.M
                self.free.append(self.ring[s][e])
                self.ring[s][e] = -1
                self.lo[s] += 1
            if self.lo[s] == self.hi[s] and self.hi[s] * self.P <= start:
                self.lo[s] = self.hi[s] = max(start, 0) // self.P
            # allocate pages up to the last new frame
            need = (end - 1) // self.P + 1
            while self.hi[s] < need:
                self.ring[s][self.hi[s] % self.M] = self.free.popleft()
                self.hi[s] += 1
            rows[b, 0] = self.appended[s]
            rows[b, 1:] = self.ring[s]
            self.appended[s] = end
        return rows

    def reset_slot(self, s: int) -> None:
        for k in range(self.lo[s], self.hi[s]):
            e = k % self.M
            self.free.append(self.ring[s][e])
            self.ring[s][e] = -1
        self.lo[s] = self.hi[s] = 0
        self.appended[s] = 0

    def reset_all(self) -> None:
        for s in range(len(self.appended)):
            self.reset_slot(s)

    def free_list(self) -> np.ndarray:
        return np.asarray(list(self.free), dtype=np.int32)

    def slot_info(self, s: int):
        return self.appended[s], np.asarray(self.ring[s], dtype=np.int32)


def _page_row(rows_b: np.ndarray, pos: int, P: int, M: int):
    page = int(rows_b[1 + (pos // P) % M])
    return page, pos % P


def append(k_pool, v_pool, rows, layer, key, value, P, M) -> None:
    """Frames key/value[b, t] go to position A_b + t of stream b (numpy)."""
    B, T, _ = key.shape
    for b in range(B):
        for t in range(T):
            page, off = _page_row(rows[b], int(rows[b, 0]) + t, P, M)
            k_pool[layer, page, off] = key[b, t]
            v_pool[layer, page, off] = value[b, t]


def gather(k_pool, v_pool, rows, layer, window, end_offset, P, M):
    """Dense window [B, window, D] of positions [A+end_offset-window, A+end_offset),
    zeros for negative positions -- the reference's view at cache.py:45."""
    B = rows.shape[0]
    D = k_pool.shape[-1]
    ok = np.zeros((B, window, D), dtype=k_pool.dtype)
    ov = np.zeros_like(ok)
    for b in range(B):
        for r in range(window):
            pos = int(rows[b, 0]) + end_offset - window + r
            if pos < 0:
                continue
            page, off = _page_row(rows[b], pos, P, M)
            ok[b, r] = k_pool[layer, page, off]
            ov[b, r] = v_pool[layer, page, off]
    return ok, ov
