"""One encoder-attention step for a batch of streams, all layers, with the
launch arguments built once.

This is the hot path of ``_encode_step`` (parakeet/engine/model_runner.py:254-304)
reduced to its paged-cache work, for serving loops that drive the kernels
directly and for measurement:

  1. open the step on the host page pool (evict / allocate) and upload, in two
     asynchronous copies from pinned memory, the batch's page rows and its
     processed_frames / cache_lengths (the reference gathers these per step with
     index_select, parakeet/engine/scheduler.py:128-170);
  2. per layer: one kernel -- fused page append + paged rel-pos attention with
     the streaming mask evaluated in the kernel from the stream state
     (attention.py:97-121, encoder.py:167-227);
  3. advance the state scalars (encoder.py:257-260) on the host mirror.

The engine always feeds whole chunks (parakeet/engine/sequence.py:137-146), so
``length`` is the chunk for every stream and the state advance is known on the
host without a device round trip.

The qkv projection output of every layer is an input ([slots, T, 3D] per
layer, q | k | v; batch row b reads row b); the outputs land in per-layer
[slots, T, D] buffers.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import ops
from ._lib import AttnArgs, check, lib
from .pool import PagePool
from .synth import Shape


class AttentionStep:
    def __init__(
        self,
        shape: Shape,
        num_slots: int,
        device: torch.device,
        qkv: list[torch.Tensor],
        pos: torch.Tensor,
        bias_u: list[torch.Tensor],
        bias_v: list[torch.Tensor],
        page_order=None,
        num_pages: int | None = None,
        rows_per_lane: int = 0,
    ):
        self.shape = shape
        self.num_slots = int(num_slots)
        self.device = device
        T, D, Ly = shape.chunk, shape.d_model, shape.layers
        self.pool = PagePool(num_slots, shape.page_size, shape.left, T, num_pages=num_pages, page_order=page_order)
        M = self.pool.max_pages
        self.k_pages = torch.empty((Ly, self.pool.num_pages, shape.page_size, D), dtype=shape.dtype, device=device)
        self.v_pages = torch.empty_like(self.k_pages)
        self.rows = torch.zeros((num_slots, 1 + M), dtype=torch.int32, device=device)
        # batch-ordered processed_frames [0, B) then cache_lengths [B, 2B)
        self.state = torch.zeros(2 * num_slots, dtype=torch.int64, device=device)
        # per-slot streaming state, advanced on the host (length == chunk)
        self.h_proc = np.zeros(num_slots, dtype=np.int64)
        self.h_cl = np.zeros(num_slots, dtype=np.int64)
        self.out = [torch.empty((num_slots, T, D), dtype=shape.dtype, device=device) for _ in range(Ly)]
        if len(qkv) != Ly or any(tuple(x.shape) != (num_slots, T, 3 * D) for x in qkv):
            raise ValueError(f"qkv must be {Ly} tensors of shape {(num_slots, T, 3 * D)}")
        self.qkv = qkv
        self.pos, self.bias_u, self.bias_v = pos, bias_u, bias_v
        # pinned staging for the per-step uploads, ring of 4: a buffer is reused
        # only after the copy that read it has completed
        depth = 4
        self._stage_rows = [torch.empty((num_slots, 1 + M), dtype=torch.int32, pin_memory=True) for _ in range(depth)]
        self._stage_state = [torch.empty(2 * num_slots, dtype=torch.int64, pin_memory=True) for _ in range(depth)]
        self._stage_ev: list[torch.cuda.Event | None] = [None] * depth
        self._stage_i = 0
        self._args = [self._attn_args(layer, rows_per_lane) for layer in range(Ly)]
        self._stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
        self.batch = 0

    # ------------------------------------------------------------ arg structs
    def _attn_args(self, layer: int, rows_per_lane: int) -> AttnArgs:
        sh = self.shape
        D = sh.d_model
        x = self.qkv[layer]
        q, k, v = x.chunk(3, dim=-1)
        pages = ops.PagedKV(self.k_pages, self.v_pages, self.rows, self.pool.max_pages)
        a = AttnArgs()
        a.dtype = ops.dtype_code(sh.dtype)
        a.device = self.device.index if self.device.index is not None else torch.cuda.current_device()
        a.pages = pages.layout()
        a.layer, a.batch, a.chunk = layer, 0, sh.chunk
        a.num_heads, a.head_dim, a.left, a.append = sh.heads, sh.head_dim, sh.left, 1
        a.query, a.query_stride_b, a.query_stride_t = q.data_ptr(), q.stride(0), q.stride(1)
        a.key, a.key_stride_b, a.key_stride_t = k.data_ptr(), k.stride(0), k.stride(1)
        a.value, a.value_stride_b, a.value_stride_t = v.data_ptr(), v.stride(0), v.stride(1)
        a.pos, a.pos_stride, a.pos_rows = self.pos.data_ptr(), self.pos.stride(0), self.pos.shape[0]
        bu, bv = self.bias_u[layer], self.bias_v[layer]
        if tuple(bu.shape) != (sh.heads, sh.head_dim) or not bu.is_contiguous() or not bv.is_contiguous():
            raise ValueError("bias_u / bias_v must be contiguous [H, dk]")
        a.bias_u, a.bias_v = bu.data_ptr(), bv.data_ptr()
        # streaming mask from the stream state (encoder.py:167-227), length == chunk
        a.processed_frames = self.state.data_ptr()
        a.cache_lengths = self.state.data_ptr()  # set per batch in run()
        a.length_scalar = sh.chunk
        a.chunk_size = sh.right + 1
        o = self.out[layer]
        a.out, a.out_stride_b, a.out_stride_t = o.data_ptr(), o.stride(0), o.stride(1)
        a.rows_per_lane = rows_per_lane
        if D != self.k_pages.shape[3]:
            raise ValueError("d_model mismatch")
        return a

    # ------------------------------------------------------------ stream life
    def reset_slots(self, slots) -> None:
        """Streams leaving (or arriving on reused slots): free their pages and
        zero their state (parakeet/engine/scheduler.py:86-91)."""
        for s in slots:
            self.pool.reset_slot(int(s))
            self.h_proc[int(s)] = 0
            self.h_cl[int(s)] = 0

    # ------------------------------------------------------------ one step
    def open(self, slots: np.ndarray) -> int:
        """Host page work + uploads for the batch ``slots``; returns B."""
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        B = int(slots.shape[0])
        if B > self.num_slots:
            raise ValueError(f"batch of {B} streams exceeds {self.num_slots} slots")
        i = self._stage_i
        self._stage_i = (i + 1) % len(self._stage_rows)
        ev = self._stage_ev[i]
        if ev is not None:
            ev.synchronize()
        rows_h = self._stage_rows[i]
        self.pool.advance(slots, out=rows_h.numpy())
        st = self._stage_state[i].numpy()
        st[:B] = self.h_proc[slots]
        st[B : 2 * B] = self.h_cl[slots]
        self.rows[:B].copy_(rows_h[:B], non_blocking=True)
        self.state[: 2 * B].copy_(self._stage_state[i][: 2 * B], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self._stage_ev[i] = ev
        # encoder.py:257-260 with length == chunk
        T = self.shape.chunk
        self.h_proc[slots] += T
        self.h_cl[slots] = np.minimum(self.h_cl[slots] + T, self.shape.left)
        self.batch = B
        return B

    def run(self, events=None) -> None:
        """All layers' fused append + attention for the batch opened last.
        ``events``: optional per-layer (start, stop) pairs timing each kernel."""
        B = self.batch
        if B == 0:
            return
        L = lib()
        cl_ptr = self.state.data_ptr() + 8 * B
        for layer, a in enumerate(self._args):
            a.batch = B
            a.cache_lengths = cl_ptr
            if events is not None:
                a.start_event, a.stop_event = events[layer]
            else:
                a.start_event = a.stop_event = None
            check(L.pk_paged_relpos_attn(ctypes.byref(a), self._stream), "pk_paged_relpos_attn")

    def step(self, slots: np.ndarray, events=None) -> None:
        self.open(slots)
        self.run(events)

    # ------------------------------------------------------------ accounting
    def bytes_per_stream(self) -> int:
        """Algorithmic HBM bytes per stream per layer: K/V window read (2L
        frames), K/V append write (2T), query read + output write (2T), the
        block-table row (4 * (1 + max_pages)) and the two state scalars (16)."""
        sh = self.shape
        s = sh.elem_bytes
        return s * sh.d_model * (2 * sh.window + 2 * sh.chunk + 2 * sh.chunk) + 4 * (1 + self.pool.max_pages) + 16

    def bytes_shared_per_launch(self) -> int:
        """Position-table rows the launch needs (left + 2T - 1) and both biases."""
        sh = self.shape
        s = sh.elem_bytes
        return s * sh.d_model * (sh.left + 2 * sh.chunk - 1) + 2 * s * sh.d_model
