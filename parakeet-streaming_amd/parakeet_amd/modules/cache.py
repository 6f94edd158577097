"""Paged drop-in for ``parakeet.modules.cache`` (parakeet/modules/cache.py).

``ModelCache`` keeps the reference constructor and methods
(``update_attn_cache``, ``get_conv_cache``, ``update_conv_cache``, ``reset``,
``reset_slot``, ``view``) but stores attention K/V in pages instead of a dense
``[N, Ly, left+right+1, D]`` shift buffer:

* ``k_pages`` / ``v_pages``: ``[Ly, num_pages, page_size, D]`` device pools
  (each page stored as 64-byte column blocks, ``ops.page_blocks``);
* a host :class:`~parakeet_amd.pool.PagePool` owns the page rings of every slot;
* each step (one pass over all layers) advances every stream of the batch by
  ``right + 1`` frames: pages that slid out of the window go back to the free
  queue, pages for the new frames are taken from it, and the batch's rows
  ``{A, ring}`` are uploaded once for all layers of the step.

A step opens lazily on the first layer update and a new one opens when a layer
is updated again, so the reference call pattern (every layer once per encoder
forward) needs no extra call.  The conv cache stays dense per slot.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass

import numpy as np
import torch
from torch import Tensor

from .. import ops
from ..pool import PagePool


class _RowStaging:
    """Pinned host buffers for the per-step row upload; a buffer is reused only
    after the copy that read it has completed, so uploads stay asynchronous."""

    def __init__(self, capacity: int, width: int, depth: int = 4):
        self.capacity = capacity
        self.width = width
        self.bufs = [torch.empty((capacity, width), dtype=torch.int32, pin_memory=True) for _ in range(depth)]
        self.events: list[torch.cuda.Event | None] = [None] * depth
        self.i = 0

    def upload(self, pool: PagePool, slots: np.ndarray, dst: Tensor) -> None:
        n = int(slots.shape[0])
        if n > self.capacity:
            self.__init__(n, self.width, len(self.bufs))
        i = self.i
        self.i = (i + 1) % len(self.bufs)
        ev = self.events[i]
        if ev is not None:
            ev.synchronize()
        buf = self.bufs[i]
        pool.advance(slots, out=buf.numpy())
        dst.copy_(buf[:n], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(dst.device))
        self.events[i] = ev


class ModelCache:
    """Paged per-stream attention cache; constructor and methods as
    parakeet/modules/cache.py:7-77.

    Extra keyword-only arguments: ``page_size`` (frames per page, power of two),
    ``num_pages`` (pool size, default ``batch_size * max_pages``) and
    ``page_order`` (initial free-queue order, default 0..num_pages-1).
    """

    def __init__(
        self,
        num_layers: int,
        attn_context_size: list | tuple,
        embed_dim: int,
        conv_kernel_size: int,
        batch_size: int = 1,
        device=None,
        dtype=None,
        *,
        page_size: int = 16,
        num_pages: int | None = None,
        page_order=None,
    ):
        super().__init__()
        self.left_attn = int(attn_context_size[0])
        self.right_attn = int(attn_context_size[1])
        self.attn_context_size = (self.left_attn, self.right_attn)
        self.attn_cache_len = self.left_attn + self.right_attn + 1
        self.conv_cache_len = int(conv_kernel_size - 1)
        self.num_layers = int(num_layers)
        self.embed_dim = int(embed_dim)
        self.chunk = self.right_attn + 1
        device = torch.device(device) if device is not None else torch.device("cpu")
        dtype = dtype if dtype is not None else torch.get_default_dtype()
        self.pool = PagePool(
            num_slots=batch_size,
            page_size=page_size,
            left=self.left_attn,
            chunk=self.chunk,
            num_pages=num_pages,
            page_order=page_order,
        )
        self.page_size = self.pool.page_size
        self.max_pages = self.pool.max_pages
        self.k_pages = torch.empty(
            (self.num_layers, self.pool.num_pages, self.page_size, self.embed_dim), device=device, dtype=dtype
        )
        self.v_pages = torch.empty_like(self.k_pages)
        # conv state per slot, frame-major: row r of [slot, layer] is column r of
        # the reference's [D, kernel-1] cache (cache.py:30-34), so a frame's
        # channels are contiguous for the fused conv step
        self.conv_frames = torch.zeros(
            (batch_size, self.num_layers, self.conv_cache_len, self.embed_dim), device=device, dtype=dtype
        )
        self._base = self
        self._staging = None
        self._set_slots(np.arange(batch_size, dtype=np.int32))

    # ------------------------------------------------------------------ views
    def _set_slots(self, slots: np.ndarray) -> None:
        self._slots = np.ascontiguousarray(slots, dtype=np.int32)
        n = int(self._slots.shape[0])
        self._prefix = bool(n == 0 or np.array_equal(self._slots, np.arange(n, dtype=np.int32)))
        dev = self._base.k_pages.device
        # uploads from pinned memory that do not wait for the GPU (torch keeps the
        # pinned buffers until the copies have run)
        def up(a):
            t = torch.from_numpy(a)
            return t.pin_memory().to(dev, non_blocking=True) if dev.type == "cuda" else t.to(dev)

        self._slot_index = None if self._prefix else up(self._slots.astype(np.int64))
        self._slots_i32 = up(self._slots.copy())
        self._rows = torch.zeros((n, 1 + self.max_pages), dtype=torch.int32, device=dev)
        self._seen: set[int] = set()
        self._step_open = False
        self._recording = False

    def _derive(self, slots: np.ndarray) -> "ModelCache":
        view = ModelCache.__new__(ModelCache)
        base = self._base
        for name in (
            "left_attn",
            "right_attn",
            "attn_context_size",
            "attn_cache_len",
            "conv_cache_len",
            "num_layers",
            "embed_dim",
            "chunk",
            "pool",
            "page_size",
            "max_pages",
            "k_pages",
            "v_pages",
            "conv_frames",
        ):
            setattr(view, name, getattr(base, name))
        view._base = base
        view._staging = None
        view._set_slots(slots)
        return view

    def view(self, batch_size: int) -> "ModelCache":
        """First ``batch_size`` rows (parakeet/modules/cache.py:65-77)."""
        if batch_size == len(self._slots):
            return self
        return self._derive(self._slots[:batch_size])

    def batch(self, slots) -> "ModelCache":
        """Cache view whose row b is pool slot ``slots[b]``; replaces the dense
        gather of Scheduler.pack_states (parakeet/engine/scheduler.py:128-170)."""
        slots = np.asarray(slots, dtype=np.int32)
        if slots.ndim != 1 or (slots.size and (slots.min() < 0 or slots.max() >= self.pool.num_slots)):
            raise ValueError(f"slots must be a 1-D list in [0, {self.pool.num_slots})")
        if len(np.unique(slots)) != len(slots):
            raise ValueError("a slot appears twice in one batch")
        return self._derive(slots)

    @property
    def batch_size(self) -> int:
        return int(self._slots.shape[0])

    @property
    def slots(self) -> np.ndarray:
        return self._slots

    # ------------------------------------------------------------------ steps
    def _begin_layer(self, layer_idx: int) -> None:
        if not 0 <= layer_idx < self.num_layers:
            raise IndexError(f"layer {layer_idx} out of range [0, {self.num_layers})")
        if self._recording:
            if layer_idx in self._seen:
                raise RuntimeError(f"paged cache: layer {layer_idx} updated twice in one recorded step")
            self._seen.add(layer_idx)
            return
        if not self._step_open or layer_idx in self._seen:
            if self._step_open and len(self._seen) != self.num_layers:
                raise RuntimeError(
                    f"paged cache: a new step began after layers {sorted(self._seen)} of "
                    f"{self.num_layers}; every layer must be updated once per step"
                )
            self._open_step()
        self._seen.add(layer_idx)

    def _open_step(self) -> None:
        base = self._base
        if self._rows.device.type == "cuda":
            if base._staging is None:
                base._staging = _RowStaging(max(1, base.pool.num_slots), 1 + self.max_pages)
            base._staging.upload(self.pool, self._slots, self._rows)
        else:
            rows = self.pool.advance(self._slots)
            self._rows.copy_(torch.from_numpy(rows))
        self._seen = set()
        self._step_open = True

    def open_step(self) -> None:
        """Opens the next step now -- the host page work for the batch and the
        upload of its rows -- instead of on the first layer update.  For callers
        that replay a recorded step, whose launches read the rows uploaded here."""
        if self._step_open and self._seen and len(self._seen) != self.num_layers:
            raise RuntimeError(
                f"paged cache: a new step began after layers {sorted(self._seen)} of {self.num_layers}"
            )
        self._open_step()

    @contextmanager
    def recording(self):
        """While recording a step (HIP graph capture), layer updates never open a
        step: the recording must hold no host work, and each replay follows an
        ``open_step()``."""
        if self._recording:
            raise RuntimeError("paged cache: already recording")
        seen = self._seen
        self._seen = set()
        self._recording = True
        try:
            yield self
        finally:
            self._recording = False
            self._seen = seen

    def paged(self) -> ops.PagedKV:
        """Device view (pools + this batch's rows) for the kernels."""
        return ops.PagedKV(self.k_pages, self.v_pages, self._rows, self.max_pages)

    def _check_chunk(self, key: Tensor, value: Tensor) -> None:
        B, T = key.shape[:2]
        if B != self.batch_size:
            raise ValueError(f"batch {B} != cache rows {self.batch_size}")
        if T != self.chunk or tuple(value.shape) != tuple(key.shape):
            raise ValueError(
                f"key/value must be [{self.batch_size}, {self.chunk}, {self.embed_dim}] "
                f"(chunk = right context + 1), got {tuple(key.shape)} / {tuple(value.shape)}"
            )

    def update_attn_cache(self, layer_idx: int, key: Tensor, value: Tensor):
        """Appends this step's frames and returns the dense window
        (K[B, L, D], V[B, L, D]) exactly as parakeet/modules/cache.py:36-45."""
        self._check_chunk(key, value)
        self._begin_layer(layer_idx)
        pages = self.paged()
        ops.kv_append(pages, layer_idx, key, value)
        return ops.kv_gather(pages, layer_idx, self.batch_size, self.attn_cache_len, self.chunk)

    def attend(
        self,
        layer_idx: int,
        query: Tensor,
        key: Tensor,
        value: Tensor,
        pos: Tensor,
        bias_u: Tensor,
        bias_v: Tensor,
        mask: Tensor | None,
        num_heads: int,
        out: Tensor | None = None,
    ) -> Tensor:
        """Fused append + paged rel-pos attention for one layer
        (parakeet/modules/attention.py:97-121 with the cache update of :97-98)."""
        self._check_chunk(key, value)
        self._begin_layer(layer_idx)
        return ops.paged_relpos_attn(
            query,
            key,
            value,
            pos,
            bias_u,
            bias_v,
            mask,
            num_heads=num_heads,
            left=self.left_attn,
            pages=self.paged(),
            layer=layer_idx,
            append=True,
            out=out,
        )

    def window(self, layer_idx: int) -> tuple[Tensor, Tensor]:
        """Dense window of the last opened step (K, V) [B, L, D], for inspection."""
        if not self._step_open:
            raise RuntimeError("no step has been opened on this cache view")
        return ops.kv_gather(self.paged(), layer_idx, self.batch_size, self.attn_cache_len, self.chunk)

    # ------------------------------------------------------------------- conv
    @property
    def conv(self) -> Tensor:
        """All slots' conv state in the reference's [N, Ly, D, kernel-1] layout
        (parakeet/modules/cache.py:30-34), as a view."""
        return self.conv_frames.transpose(2, 3)

    def get_conv_cache(self, layer_idx: int) -> Tensor:
        """[B, D, kernel-1] conv state of this batch (cache.py:47-48)."""
        if self._prefix:
            return self.conv_frames[: self.batch_size, layer_idx].transpose(1, 2)
        return self.conv_frames[self._slot_index, layer_idx].transpose(1, 2)

    def update_conv_cache(self, layer_idx: int, state: Tensor) -> None:
        """Stores a [B, D, kernel-1] conv state (cache.py:50-53); None is a no-op,
        which is what the fused step returns after updating the cache in place."""
        if state is None:
            return
        frames = state.transpose(1, 2)
        if self._prefix:
            self.conv_frames[: self.batch_size, layer_idx].copy_(frames)
        else:
            self.conv_frames[self._slot_index, layer_idx] = frames.to(self.conv_frames.dtype)

    def conv_ref(self, layer_idx: int) -> "ConvCacheRef":
        """Handle that makes ConformerConvolution.forward update this batch's conv
        state in place (the fused step) instead of returning a new state."""
        if not 0 <= layer_idx < self.num_layers:
            raise IndexError(f"layer {layer_idx} out of range [0, {self.num_layers})")
        return ConvCacheRef(self, int(layer_idx))

    def conv_step(
        self,
        layer_idx: int,
        glu_in: Tensor,
        pad_mask: Tensor | None,
        dw_weight: Tensor,
        dw_bias: Tensor | None,
        ln_weight: Tensor,
        ln_bias: Tensor,
        eps: float,
    ) -> Tensor:
        """GLU -> pad mask -> causal depthwise conv over [state ; frames] ->
        LayerNorm -> SiLU for this batch, the state of each stream's slot updated
        in place (convolution.py:37-47,152-157 with cache.py:47-53)."""
        if glu_in.shape[0] != self.batch_size:
            raise ValueError(f"batch {glu_in.shape[0]} != cache rows {self.batch_size}")
        return ops.conv_step(
            glu_in,
            self.conv_frames,
            dw_weight,
            ln_weight,
            ln_bias,
            layer=layer_idx,
            slots=None if self._prefix else self._slots_i32,
            pad_mask=pad_mask,
            dw_bias=dw_bias,
            eps=eps,
        )

    # ------------------------------------------------------------------ reset
    def reset(self) -> None:
        """All slots empty (parakeet/modules/cache.py:55-58)."""
        self.pool.reset_all()
        self.conv_frames.zero_()
        self._step_open = False
        self._seen = set()

    def reset_slot(self, slot: int) -> None:
        """Row ``slot`` empty: its pages go back to the pool and its window reads
        as zeros again (parakeet/modules/cache.py:60-63)."""
        pool_slot = int(self._slots[slot])
        self.pool.reset_slot(pool_slot)
        self.conv_frames[pool_slot].zero_()


@dataclass
class ConvCacheRef:
    """One layer of a batch's conv state, updated in place by the fused step."""

    cache: ModelCache
    layer_idx: int


@dataclass
class StreamingState:
    """Per-batch streaming state (parakeet/modules/cache.py:80-89)."""

    cache: ModelCache
    processed_frames: Tensor | int = 0
    cache_lengths: Tensor | int = 0

    def attn_cache_len(self) -> int:
        if isinstance(self.cache_lengths, Tensor):
            return int(self.cache_lengths.max().item())
        return int(self.cache_lengths)


__all__ = ["ConvCacheRef", "ModelCache", "StreamingState"]
