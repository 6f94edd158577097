"""Drop-in for ``parakeet.engine.scheduler`` (parakeet/engine/scheduler.py).

Admission (``add``/``admit_ready``/``release``) and the slot pool
(``init_state_pool``/``acquire_state_slot``/``release_state_slot``) keep the
reference's deques and locks.  ``pack_states``/``unpack_states`` no longer copy
the dense K/V/conv state of every stream in and out of a batch buffer
(scheduler.py:128-201): the batch is a view of the paged cache whose rows are
the streams' slots, and only the two int64 state scalars are gathered and
scattered.  K/V pages are written in place by the kernels.

Sequences are duck-typed: any object with ``status`` (an enum with members named
WAITING/RUNNING/FINISHED) and ``encoder_state`` (slot id) works, including the
reference's ``parakeet.engine.sequence.Sequence``.
"""

from __future__ import annotations

import threading
from collections import deque
from dataclasses import dataclass
from enum import Enum, auto
from typing import Deque, Iterable

import torch

from ..modules.cache import StreamingState


class SequenceStatus(Enum):
    """Same members as parakeet/engine/sequence.py:10-13."""

    WAITING = auto()
    RUNNING = auto()
    FINISHED = auto()


def _status(seq) -> str:
    return getattr(seq.status, "name", str(seq.status))


def _set_status(seq, name: str) -> None:
    cls = type(seq.status) if isinstance(seq.status, Enum) else SequenceStatus
    seq.status = cls[name]


@dataclass
class StreamResult:
    stream_id: int
    text: str
    token_ids: list[int]
    is_final: bool


class Scheduler:
    """Stream admission plus the paged state pool (parakeet/engine/scheduler.py:20-201)."""

    def __init__(self, max_active: int = 64):
        self.max_active = max_active
        self.waiting: Deque = deque()
        self.active: Deque = deque()
        self._lock = threading.Lock()
        self._state_lock = threading.Lock()
        self._pool_state: StreamingState | None = None
        self._free_slots: Deque[int] = deque()
        self._state_encoder = None
        self._state_device: torch.device | None = None
        self._state_dtype: torch.dtype | None = None

    # ---------------------------------------------------------- admission
    def add(self, seq) -> None:
        with self._lock:
            if len(self.active) < self.max_active:
                _set_status(seq, "RUNNING")
                self.active.append(seq)
            else:
                _set_status(seq, "WAITING")
                self.waiting.append(seq)

    def admit_ready(self) -> list:
        admitted = []
        with self._lock:
            while self.waiting and len(self.active) < self.max_active:
                seq = self.waiting.popleft()
                if _status(seq) == "FINISHED":
                    continue
                _set_status(seq, "RUNNING")
                self.active.append(seq)
                admitted.append(seq)
        return admitted

    def release(self, seq) -> None:
        with self._lock:
            if seq in self.waiting:
                self.waiting.remove(seq)
            if seq in self.active:
                self.active.remove(seq)
            _set_status(seq, "FINISHED")

    def active_sequences(self) -> Iterable:
        with self._lock:
            return list(self.active)

    # ---------------------------------------------------------- state pool
    def init_state_pool(self, encoder, device: torch.device, dtype: torch.dtype, pool_size: int, **cache_kwargs) -> None:
        """Pool of ``pool_size`` slots; ``cache_kwargs`` (page_size, num_pages,
        page_order) go to the paged ModelCache."""
        with self._state_lock:
            self._state_encoder = encoder
            self._state_device = device
            self._state_dtype = dtype
            self._pool_state = encoder.init_streaming_state(
                batch_size=pool_size, device=device, dtype=dtype, **cache_kwargs
            )
            self._free_slots = deque(range(pool_size))

    @property
    def pool_state(self) -> StreamingState | None:
        return self._pool_state

    def _reset_state(self, slot: int) -> None:
        if self._pool_state is None:
            return
        self._pool_state.processed_frames[slot : slot + 1].zero_()
        self._pool_state.cache_lengths[slot : slot + 1].zero_()
        self._pool_state.cache.reset_slot(slot)

    def acquire_state_slot(self) -> int | None:
        with self._state_lock:
            if not self._free_slots:
                return None
            slot = self._free_slots.popleft()
        self._reset_state(slot)
        return slot

    def release_state_slot(self, slot: int) -> None:
        self._reset_state(slot)
        with self._state_lock:
            self._free_slots.append(slot)

    # ---------------------------------------------------------- batches
    def pack_states(self, seqs: Iterable) -> tuple[StreamingState, torch.Tensor]:
        """Batch state for ``seqs``: a cache view over their slots plus the
        gathered processed_frames / cache_lengths."""
        if self._pool_state is None:
            raise RuntimeError("State pool not initialized.")
        seqs = list(seqs)
        slot_ids = [seq.encoder_state for seq in seqs]
        # from pinned memory, without waiting for the GPU (torch keeps the pinned
        # buffer until the copy has run)
        slot_index = torch.tensor(slot_ids, dtype=torch.long)
        dev = torch.device(self._state_device)
        slot_index = slot_index.pin_memory().to(dev, non_blocking=True) if dev.type == "cuda" else slot_index.to(dev)
        pool = self._pool_state
        state = StreamingState(
            cache=pool.cache.batch(slot_ids),
            processed_frames=torch.index_select(pool.processed_frames, 0, slot_index),
            cache_lengths=torch.index_select(pool.cache_lengths, 0, slot_index),
        )
        return state, slot_index

    def unpack_states(self, batch_state: StreamingState, slot_index: torch.Tensor) -> None:
        if self._pool_state is None:
            return
        self._pool_state.processed_frames.index_copy_(0, slot_index, batch_state.processed_frames)
        self._pool_state.cache_lengths.index_copy_(0, slot_index, batch_state.cache_lengths)


__all__ = ["Scheduler", "SequenceStatus", "StreamResult"]
