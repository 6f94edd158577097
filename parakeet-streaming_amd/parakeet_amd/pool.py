"""Host page pool: FIFO free-page queue and per-slot page rings (C++ side).

Replaces the reference's slot pool / dense shift buffers
(parakeet/engine/scheduler.py:68-104, parakeet/modules/cache.py:8-63): a slot
owns a ring of ``max_pages`` page ids; each step frees the pages that slid out
of its window and allocates pages for the new frames.
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_int32, c_int64, c_void_p

import numpy as np

from ._lib import check, lib


def pages_per_slot(left: int, chunk: int, page_size: int) -> int:
    """Ring entries a slot needs: a window of left+chunk frames touches at most
    (window + page_size - 2) // page_size + 1 pages."""
    window = left + chunk
    return (window + page_size - 2) // page_size + 1


def _i32p(a: np.ndarray):
    return a.ctypes.data_as(POINTER(c_int32))


class PagePool:
    """Thread-safe page allocator; every call goes to ``pk_pool_*``."""

    def __init__(
        self,
        num_slots: int,
        page_size: int,
        left: int,
        chunk: int,
        num_pages: int | None = None,
        page_order=None,
    ):
        self.num_slots = int(num_slots)
        self.page_size = int(page_size)
        self.left = int(left)
        self.chunk = int(chunk)
        self.max_pages = pages_per_slot(self.left, self.chunk, self.page_size)
        if num_pages is None:
            num_pages = self.num_slots * self.max_pages
        self.num_pages = int(num_pages)
        self.rows_stride = 1 + self.max_pages
        order_ptr = None
        if page_order is not None:
            order = np.ascontiguousarray(np.asarray(page_order, dtype=np.int32))
            if order.shape != (self.num_pages,):
                raise ValueError(f"page_order must have {self.num_pages} entries, got {order.shape}")
            self._order = order
            order_ptr = _i32p(order)
        handle = c_void_p()
        check(
            lib().pk_pool_create(
                self.num_pages,
                self.num_slots,
                self.page_size,
                self.left,
                self.chunk,
                order_ptr,
                ctypes.byref(handle),
            ),
            "pk_pool_create",
        )
        self._h = handle
        got = lib().pk_pool_max_pages(self._h)
        if got != self.max_pages:
            raise RuntimeError(f"pk_pool_max_pages {got} != {self.max_pages}")

    # -- lifetime
    def close(self) -> None:
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib().pk_pool_destroy(h)
            self._h = c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- stepping
    def advance(self, slots: np.ndarray, out: np.ndarray | None = None) -> np.ndarray:
        """Opens one step for ``slots`` (in order): evicts, allocates, returns
        int32 rows [n, 1 + max_pages] = {A, ring...} and advances each A by chunk."""
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        n = int(slots.shape[0])
        if out is None:
            out = np.empty((n, self.rows_stride), dtype=np.int32)
        if out.dtype != np.int32 or not out.flags.c_contiguous or out.shape[0] < n or out.shape[1] != self.rows_stride:
            raise ValueError("advance: out must be C-contiguous int32 [n, 1 + max_pages]")
        check(lib().pk_pool_advance(self._h, n, _i32p(slots), _i32p(out), self.rows_stride), "pk_pool_advance")
        return out[:n]

    def reset_slot(self, slot: int) -> None:
        check(lib().pk_pool_reset_slot(self._h, int(slot)), "pk_pool_reset_slot")

    def reset_all(self) -> None:
        check(lib().pk_pool_reset_all(self._h), "pk_pool_reset_all")

    # -- inspection
    def free_pages(self) -> int:
        return check(lib().pk_pool_free_pages(self._h), "pk_pool_free_pages")

    def free_list(self) -> np.ndarray:
        n = self.free_pages()
        out = np.empty(max(n, 1), dtype=np.int32)
        got = check(lib().pk_pool_free_list(self._h, _i32p(out), out.shape[0]), "pk_pool_free_list")
        return out[:got].copy()

    def slot_info(self, slot: int) -> tuple[int, np.ndarray]:
        appended = c_int64()
        ring = np.empty(self.max_pages, dtype=np.int32)
        check(
            lib().pk_pool_slot_info(self._h, int(slot), ctypes.byref(appended), _i32p(ring)),
            "pk_pool_slot_info",
        )
        return int(appended.value), ring
